"""GPU parity of page selection and block-sparse attention against the oracle,
on the benchmark's synthetic workloads (small sizes in full, 32K on sampled rows
plus size-independent plan invariants)."""
import dataclasses

import pytest
import torch

import oracle
from gpu_helpers import oracle_select_rows, plan_structure_errors, spread_rows
from leanselect_amd import _hip, workloads
from leanselect_amd.ops import compress_k, leanselect_prefill_topk_idx, sparse_attention
from leanselect_amd.ops.attention import attention_tile_rows, infllmv2_attn_varlen_func
from leanselect_amd.ops.nosa import nosa_sparse_attention
from leanselect_amd.prefill import leanselect_sparse_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _select(case):
    kc, cu_c = compress_k(case.k, case.cu_seqlens, cu_seqlens_host=case.cu_host)
    ids = leanselect_prefill_topk_idx(
        case.q, kc, case.cu_seqlens, cu_c, case.selector, topk=case.topk,
        init_blocks=case.init_blocks, local_blocks=case.local_blocks, cu_seqlens_q_host=case.cu_host)
    return kc, cu_c, ids


def _check_select(case, rows=None):
    kc, cu_c, ids = _select(case)
    take = ids.shape[-1]
    errs = plan_structure_errors(ids, case.cu_host, take, case.init_blocks, case.local_blocks)
    assert not errs, errs
    kc_cpu = kc.cpu()
    want_kc, want_cu = oracle.compress_k(case.k.cpu(), case.cu_host)
    assert cu_c.cpu().tolist() == want_cu.tolist()
    if case.q.dtype == torch.float32:
        torch.testing.assert_close(kc_cpu, want_kc, rtol=2e-6, atol=1e-6)
    # Parity of the plans uses the GPU's compressed keys so the rows test selection alone.
    want_ids, scores = oracle_select_rows(case, kc_cpu, cu_c.cpu().tolist(), rows, case.q.dtype)
    got = ids.cpu() if rows is None else ids.cpu()[:, rows]
    rep = oracle.check_topk(got, want_ids, scores, case.q.dtype)
    print(f"\nselect parity: {rep}")
    assert rep.ok, str(rep)
    return kc, cu_c, ids, rep


def test_select_head_space_fp32_4k():
    case = workloads.head_space_layer(4096, device=DEV)
    _, _, ids, rep = _check_select(case)
    assert ids.shape == (2, 4096, 16)
    assert rep.exact_rows == rep.rows  # float32: every row bit-exact


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_select_hidden_space_4k(dtype):
    case = workloads.hidden_space_layer((4096,), device=DEV, dtype=dtype, seed=1)
    _, _, ids, rep = _check_select(case)
    assert ids.shape == (2, 4096, 64)
    assert rep.exact_rows == rep.rows and rep.band_rows == 0


@pytest.mark.parametrize("router", [(8, 32), (2, 32), (3, 32)])
def test_select_router_widths(router):
    # F = 256 takes the scoring kernel with the shared LDS panel at 8 k-slices;
    # F = 64 and 96 take the per-wave kernel (the panel needs 16 or 32 chunks a row).
    rh, rd = router
    case = workloads.hidden_space_layer((4096,), device=DEV, dtype=torch.bfloat16, seed=2,
                                        router_heads=rh, router_dim=rd)
    _, _, ids, rep = _check_select(case)
    assert ids.shape == (2, 4096, 64)
    assert rep.exact_rows == rep.rows and rep.band_rows == 0


def test_select_ragged_with_short_sequences():
    lens = (8, 31, 32, 100, 1000, 2113, 64, 0, 4500)
    case = workloads.hidden_space_layer(lens, device=DEV, seed=2)
    _, _, ids, rep = _check_select(case)
    cu = case.cu_host
    # Sequences shorter than one compression window get no plan at all.
    for b, n in enumerate(lens):
        if 0 < n < 32:
            assert bool((ids[:, cu[b] : cu[b + 1]] == -1).all())


def test_batch_without_any_compressed_key():
    """Every sequence shorter than one compression window: no compressed key in the
    whole batch, so no page for any row (the reference skips such sequences,
    minicpm.py:3115-3116) and a zero attention output."""
    lens = (8, 31, 1)
    case = workloads.hidden_space_layer(lens, device=DEV, seed=4)
    kc, cu_c, ids = _select(case)
    assert kc.shape[0] == 0 and cu_c.cpu().tolist() == [0, 0, 0, 0]
    assert ids.shape == (2, sum(lens), 1) and bool((ids == -1).all())
    out, ids2 = leanselect_sparse_prefill(
        case.q, case.k, case.v, case.cu_seqlens, case.selector, topk=case.topk,
        local_blocks=case.local_blocks, init_blocks=case.init_blocks,
        cu_seqlens_host=case.cu_host, return_topk_idx=True)
    torch.cuda.synchronize()
    assert torch.equal(ids2, ids) and not bool(out.any())


def test_select_rows_with_nonpositive_kth_scores():
    """bf16 rows take a fast top-k path only while their kk-th score is positive
    (reads past the row come back as +0); rows whose kk-th score is zero or
    negative take the general path.  The keys are shifted along one direction,
    so most of a row's scores share the sign of q~ . shift, and some query rows
    are zero (every score +0, all tied).  Long rows of both kinds must match the
    oracle."""
    case = workloads.hidden_space_layer((32768,), hidden=1024, device=DEV, seed=41)
    gen = torch.Generator(device="cpu").manual_seed(5)
    shift = (torch.randn(case.k.shape[1:], generator=gen) * 20.0).to(DEV)
    k = (case.k.float() + shift).to(case.k.dtype)
    q = case.q.clone()
    zero_rows = [20000, 20001, 31000]
    q[zero_rows] = 0
    case = dataclasses.replace(case, q=q, k=k)
    rows = sorted(set(spread_rows(case.cu_host, per_seq=96)) | set(zero_rows))
    kc, cu_c, ids = _select(case)
    want, scores = oracle_select_rows(case, kc.cpu(), cu_c.cpu().tolist(), rows, case.q.dtype)
    rep = oracle.check_topk(ids.cpu()[:, rows], want, scores, case.q.dtype)
    print(f"\nselect parity (shifted keys): {rep}")
    assert rep.ok, str(rep)
    take = ids.shape[-1]
    pos = nonpos = 0
    for g in range(scores.shape[0]):
        for i in range(len(rows)):
            s = scores[g, i]
            fin = s[torch.isfinite(s)]
            n_forced = int(torch.isposinf(s).sum())
            kk = min(take, n_forced + fin.numel()) - n_forced
            if fin.numel() <= 256 or kk < 1:
                continue  # rows of up to four slots always take the general path
            kth = float(fin.sort(descending=True).values[kk - 1])
            pos += kth > 0
            nonpos += kth <= 0
    print(f"long rows with a positive kk-th score: {pos}, zero or negative: {nonpos}")
    assert pos >= 10 and nonpos >= 10


def test_select_rows_of_tied_scores():
    """Every key row equal, so every page of a row scores the same: rows whose
    score is positive pass the fast path's bound but gather more than 256 ties
    (the general path takes over), the others fail the bound.  Ties go to the
    lowest pages."""
    case = workloads.hidden_space_layer((24576,), hidden=1024, device=DEV, seed=43)
    k = case.k[:1].expand_as(case.k).contiguous()
    case = dataclasses.replace(case, k=k)
    rows = spread_rows(case.cu_host, per_seq=96)
    _, _, ids, rep = _check_select(case, rows=rows)
    assert rep.exact_rows == rep.rows
    # The chosen non-forced pages are the lowest ones: 1, 2, ... (sink page 0).
    for r in rows:
        qp = r // 64
        if qp > case.topk:
            assert ids[0, r, : case.topk - 5].tolist() == list(range(case.topk - 5))


def test_select_32k_sampled_rows():
    case = workloads.hidden_space_layer((32768,), device=DEV, seed=3)
    rows = spread_rows(case.cu_host, per_seq=128)
    _, _, ids, rep = _check_select(case, rows=rows)
    assert rep.exact_rows == rep.rows and rep.band_rows == 0


def test_select_128k_sampled_rows():
    """Every per-row slot count of the 128K layer (1..32 slots of 64 candidates)."""
    case = workloads.hidden_space_layer((131072,), device=DEV, seed=5)
    rows = spread_rows(case.cu_host, per_seq=96)
    _, _, ids, rep = _check_select(case, rows=rows)
    assert rep.exact_rows == rep.rows and rep.band_rows == 0


def test_select_300k_ragged_widest_slots():
    """Candidate rows longer than 4096 pages (128 register slots) next to a short sequence."""
    case = workloads.hidden_space_layer((300000, 5000), device=DEV, seed=6)
    rows = spread_rows(case.cu_host, per_seq=48)
    _, _, ids, rep = _check_select(case, rows=rows)
    assert rep.exact_rows == rep.rows and rep.band_rows == 0


def test_select_fp32_160k_sampled_rows():
    """float32 scores (32-bit keys) with 64 register slots; float32 rows are bit-exact."""
    case = workloads.head_space_layer(160000, device=DEV, seed=7)
    rows = spread_rows(case.cu_host, per_seq=64)
    _, _, ids, rep = _check_select(case, rows=rows)
    assert rep.exact_rows == rep.rows


def _attention_case(dtype=torch.bfloat16, lens=(3000,), seed=4, **kw):
    case = workloads.hidden_space_layer(lens, device=DEV, dtype=dtype, seed=seed, **kw)
    _, _, ids = _select(case)
    return case, ids


def _check_attention(case, ids, rows, **kw):
    out, lse = sparse_attention(case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens,
                                case.max_seqlen, case.max_seqlen, ids, return_lse=True, **kw)
    want, want_lse = oracle.sparse_attention(
        case.q.cpu(), case.k.cpu(), case.v.cpu(), case.cu_host, case.cu_host,
        ids.cpu()[:, rows], rows=rows, ids_rows_aligned=True, **kw)
    ok, mx, mr = oracle.check_attention(out.cpu()[rows], want)
    print(f"\nattention parity: max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert ok, (mx, mr)
    got_lse = lse.cpu()[:, rows]
    fin = torch.isfinite(want_lse)
    assert torch.equal(torch.isfinite(got_lse), fin)
    torch.testing.assert_close(got_lse[fin], want_lse[fin], rtol=1e-4, atol=2e-3)
    return out


def test_attention_matches_oracle_bf16():
    case, ids = _attention_case()
    rows = spread_rows(case.cu_host, per_seq=64)
    _check_attention(case, ids, rows)


def test_attention_fp16_and_scale():
    case, ids = _attention_case(dtype=torch.float16, seed=5)
    rows = spread_rows(case.cu_host, per_seq=48)
    _check_attention(case, ids, rows, softmax_scale=0.05)


def test_attention_ragged_batch():
    case, ids = _attention_case(lens=(1, 31, 65, 700, 2000), seed=6)
    rows = spread_rows(case.cu_host, per_seq=40)
    out = _check_attention(case, ids, rows)
    # Rows without any page (sequences shorter than a compression window) are zero.
    assert bool((out[:32] == 0).all())


def test_attention_every_row_of_a_ragged_batch():
    """Every row of a batch whose tile count (24-row tiles per sequence, 64-id plans)
    is far from a multiple of the launch's rounding: each tile index reaches exactly
    one workgroup of the XCD-dealt grid, and surplus workgroups exit without writing."""
    case, ids = _attention_case(lens=(700, 1300, 64, 17, 2500, 333), seed=8)
    _check_attention(case, ids, list(range(case.cu_host[-1])))


def test_attention_messy_ids_duplicates_unsorted_out_of_range():
    case, ids = _attention_case(lens=(1500,), seed=7)
    g = torch.Generator(device="cpu").manual_seed(0)
    G, N, T = ids.shape
    messy = torch.randint(-3, 30, (G, N, T), generator=g, dtype=torch.int32)
    messy[..., 0] = messy[..., 1]  # duplicates
    rows = spread_rows(case.cu_host, per_seq=40)
    _check_attention(case, messy.to(DEV), rows)


@pytest.mark.parametrize("take,dtype,N", [(85, torch.bfloat16, 131072),
                                          (96, torch.bfloat16, 147456),
                                          (128, torch.float16, 196608)])
def test_attention_tile_unions_at_their_bound(take, dtype, N):
    """Row r of a 24-row tile takes pages r*take .. r*take + take - 1 (mod the visible
    pages), so at the end of an N-token sequence no two rows of a tile share a page
    and the last full tile's union holds 24 x take pages: 2040, 2304 and 3072 (the
    bound of the 128-id plans the kernel accepts, past the 2048 pages of a 32-bit
    need word per lane); earlier rows repeat ids, which the kernel drops."""
    case = workloads.hidden_space_layer((N,), device=DEV, dtype=dtype, seed=31)
    G = case.k.shape[1]
    tile = attention_tile_rows(take)
    assert tile == 24
    t = torch.arange(N, dtype=torch.int64)
    visible = (t // 64 + 1)[:, None]
    base = (t % tile)[:, None] * take + torch.arange(take, dtype=torch.int64)[None, :]
    ids = torch.stack([(base + 977 * g) % visible for g in range(G)]).to(torch.int32)
    last = (N // tile - 1) * tile
    for g in range(G):
        assert ids[g, last : last + tile].unique().numel() == tile * take
    rows = sorted(set(spread_rows(case.cu_host, per_seq=24)) |
                  set(range(last - tile, last + tile)) | set(range(N - 8, N)))
    _check_attention(case, ids.to(DEV), rows)


@pytest.mark.parametrize("take", [0, 5])
def test_attention_plans_without_pages(take):
    """Plans with no ids (take 0) or only -1 ids: no union page, so every row's
    output is zero and its log-sum-exp +inf (flash attention's empty-row rule),
    and no wait of the ring is entered."""
    case = workloads.hidden_space_layer((700, 300), device=DEV, seed=12)
    G, N = case.k.shape[1], case.cu_host[-1]
    ids = torch.full((G, N, take), -1, dtype=torch.int32, device=DEV)
    out, lse = sparse_attention(case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens,
                                case.max_seqlen, case.max_seqlen, ids, return_lse=True,
                                sync_status=True)
    assert bool((out == 0).all())
    assert bool(torch.isposinf(lse).all())


def test_attention_union_sizes_with_small_factors():
    """Tiles whose union has 1, 2, 7, 14, 21, 35 or 49 pages (the visit order is a
    stride permutation of the union, which must stay a bijection for every size)."""
    case, ids = _attention_case(lens=(4096,), seed=10)
    G, N, T = ids.shape
    tile = attention_tile_rows(T)
    crafted = torch.full((G, N, T), -1, dtype=torch.int32)
    sizes = [1, 2, 7, 14, 21, 35, 49]
    for t in range(N):
        k = sizes[(t // tile) % len(sizes)]
        pages = [p for p in range(k) if p <= t // 64][:T]
        crafted[:, t, : len(pages)] = torch.tensor(pages, dtype=torch.int32)
    rows = spread_rows(case.cu_host, per_seq=64)
    _check_attention(case, crafted.to(DEV), rows)


def test_attention_group_size_4_and_non_causal():
    case = workloads.head_space_layer(1024, device=DEV, dtype=torch.bfloat16)
    _, _, ids = _select(case)
    rows = spread_rows(case.cu_host, per_seq=40)
    _check_attention(case, ids, rows)
    _check_attention(case, ids, rows, causal=False)


def test_infllm_surface_returns_lse_tuple():
    case, ids = _attention_case(lens=(700,), seed=8)
    out = infllmv2_attn_varlen_func(case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens,
                                    700, 700, causal=True, topk_idx=ids)
    out2, lse, s = infllmv2_attn_varlen_func(case.q, case.k, case.v, case.cu_seqlens,
                                             case.cu_seqlens, 700, 700, causal=True,
                                             return_attn_probs=True, topk_idx=ids)
    assert torch.equal(out, out2) and lse.shape == (32, 700) and s.numel() == 0


def test_end_to_end_prefill_32k_sampled():
    case = workloads.hidden_space_layer((32768,), device=DEV, seed=9)
    out, ids = leanselect_sparse_prefill(
        case.q, case.k, case.v, case.cu_seqlens, case.selector, topk=case.topk,
        local_blocks=case.local_blocks, init_blocks=case.init_blocks,
        cu_seqlens_host=case.cu_host, return_topk_idx=True)
    assert not plan_structure_errors(ids, case.cu_host, 64, 1, 4)
    rows = spread_rows(case.cu_host, per_seq=24)
    want, _ = oracle.sparse_attention(case.q.cpu(), case.k.cpu(), case.v.cpu(), case.cu_host,
                                      case.cu_host, ids.cpu()[:, rows], rows=rows,
                                      ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(out.cpu()[rows], want)
    assert ok, (mx, mr)


def test_ring_wait_expiry_is_reported():
    """With the wait bound forced to zero from the host every ring wait expires at
    once: the kernel still finishes, the status word is set and the wrapper raises
    (at once with ``sync_status``; at ``attn_status_sync`` otherwise, without the
    call itself waiting), and the rows of the waves whose wait expired are NaN.
    The next call with the default bound is clean and correct."""
    case, ids = _attention_case(lens=(3000,), seed=4)
    L = _hip.lib()
    out = torch.zeros_like(case.q)
    _hip.attn_status_sync()  # nothing earlier is pending
    L.ls_attn_set_spin_limit(0)
    try:
        with pytest.raises(RuntimeError, match="expired"):
            sparse_attention(case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens,
                             3000, 3000, ids, out=out, sync_status=True)
        out2 = torch.zeros_like(case.q)
        sparse_attention(case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens,
                         3000, 3000, ids, out=out2)  # deferred: returns without raising
        with pytest.raises(RuntimeError, match="expired"):
            _hip.attn_status_sync()
    finally:
        L.ls_attn_set_spin_limit(-1)
    _hip.attn_status_sync()  # the queue is drained
    nan_rows = torch.isnan(out.float()).any(dim=2).any(dim=1)
    assert bool(nan_rows.any())
    # a row is either NaN in every head of a group or has finite values there
    per_group = torch.isnan(out.float()).any(dim=2).view(out.shape[0], 2, -1)
    assert bool((per_group.all(dim=2) == per_group.any(dim=2)).all())
    rows = spread_rows(case.cu_host, per_seq=32)
    _check_attention(case, ids, rows)
    _hip.attn_status_sync()


def test_empty_attention_calls_read_no_stale_status():
    """Calls with no query rows (or no sequences) launch no kernel, so they must
    not read a status word: the workspace then holds whatever the allocator's
    reused block held.  A freed block of 0xFF bytes comes first."""
    junk = torch.full((1 << 20,), 255, dtype=torch.uint8, device=DEV)
    del junk
    G, H, D = 2, 8, 128
    q = torch.empty(0, H, D, dtype=torch.bfloat16, device=DEV)
    k = torch.randn(128, G, D, device=DEV).to(torch.bfloat16)
    v = torch.randn(128, G, D, device=DEV).to(torch.bfloat16)
    ids = torch.empty(G, 0, 4, dtype=torch.int32, device=DEV)
    cu_q = torch.zeros(2, dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0, 128], dtype=torch.int32, device=DEV)
    out = sparse_attention(q, k, v, cu_q, cu_k, 0, 128, ids, sync_status=True)
    assert out.shape == (0, H, D)
    out = nosa_sparse_attention(q, k, v, torch.zeros(128, G, device=DEV), cu_q, cu_k, 0, 128,
                                ids, sync_status=True)
    assert out.shape == (0, H, D)
    none = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = sparse_attention(q, k, v, none, none, 0, 0, ids, sync_status=True)
    assert out.shape == (0, H, D)
    _hip.attn_status_sync()


def test_prefill_step_graph_replays_match_eager():
    """The whole step (compressed keys, selection, attention), with the host
    offsets given, captured in one HIP graph: three replays, with an eager step
    between them, each giving the eager step's plans and output bit for bit."""
    case = workloads.hidden_space_layer((2500, 1100), device=DEV, seed=12)

    def step():
        return leanselect_sparse_prefill(
            case.q, case.k, case.v, case.cu_seqlens, case.selector, topk=case.topk,
            local_blocks=case.local_blocks, init_blocks=case.init_blocks,
            cu_seqlens_host=case.cu_host, return_topk_idx=True)

    want_out, want_ids = step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, ids_g = step()
    for _ in range(3):
        out_g.zero_()
        ids_g.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids_g, want_ids)
        assert torch.equal(out_g, want_out)
        out_e, ids_e = step()
        assert torch.equal(ids_e, want_ids) and torch.equal(out_e, want_out)


def test_sparse_attention_graph_replays_match_eager():
    """The attention call captured in a HIP graph (workspace and plans formed by
    kernels, no memset nodes, no host read under capture): three replays, with
    eager calls and a clear of the output between them, each equal to the eager
    result bit for bit."""
    case, ids = _attention_case(lens=(3000, 1300), seed=6)
    args = (case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens, 3000, 3000, ids)
    want = sparse_attention(*args)
    out = torch.empty_like(want)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sparse_attention(*args, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sparse_attention(*args, out=out)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        assert torch.equal(sparse_attention(*args), want)
