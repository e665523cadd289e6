"""GPU parity of the NOSA variant against the oracle: CIS mean pooling, the
varlen page max-pool, the fused two-stage selection and the CIS-biased
attention.

The fused selection is compared in two ways: bit-exactly against the oracle's
selection run on the GPU's own intermediate scores (qk page scores from
``score_pages`` and CIS window means from ``nosa_mean_pooling``, which run the
same arithmetic as the fused kernels), and row by row against the fully
independent oracle, where only rows with near-tied scores may differ."""
import pytest
import torch

import oracle
from gpu_helpers import spread_rows
from leanselect_amd import workloads
from leanselect_amd.ops import (compress_k, max_pooling_1d_varlen, nosa_mean_pooling,
                                nosa_prefill_topk_idx, nosa_sparse_attention, sparse_attention)
from leanselect_amd.prefill import nosa_sparse_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cis(total, G, dtype=torch.bfloat16, seed=0, std=1.0):
    g = torch.Generator(device="cpu").manual_seed(1000 + seed)
    return (torch.randn(total, G, generator=g) * std).to(dtype)


# ---------------------------------------------------------------------------
# CIS mean pooling and the varlen page max-pool
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_cis_mean_pooling(dtype):
    lens = [5, 31, 32, 33, 100, 0, 1000, 2113]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    cis = _cis(cu[-1], 3, dtype, seed=1)
    got = nosa_mean_pooling(cis.to(DEV), torch.tensor(cu, dtype=torch.int32, device=DEV),
                            max(lens)).cpu()
    want = oracle.nosa_mean_pooling(cis, cu, max(lens))
    assert got.shape == want.shape == (3, cu[-1], max(lens) // 16 - 1)
    # float32 sums of 32 values, rounded once: within one step of the exact mean.
    tol = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 1e-6}[dtype]
    torch.testing.assert_close(got.double(), want.double(), rtol=tol, atol=1e-6)
    exact = (got == want).double().mean().item()
    print(f"\nmean pooling exact fraction {exact:.5f}")
    if dtype != torch.float32:  # a 16-bit rounding hides the summation order
        assert exact >= 0.99
    # Windows that do not fit in their sequence are 0.
    for b, n in enumerate(lens):
        m_fit = max(0, (n - 32) // 16 + 1) if n >= 32 else 0
        assert bool((got[:, cu[b] : cu[b + 1], m_fit:] == 0).all())


@pytest.mark.parametrize("clip", ["sequence", "row"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_page_maxpool_varlen_exact(dtype, clip):
    """Every score column holds a value (the padding too), so the two clips
    give different pages wherever a shorter sequence's window reaches past its
    columns."""
    lens_q, lens_k, cache = [700, 1, 130, 2000], [40, 0, 7, 124], [0, 128, 5, 0]
    cq, ck = [0], [0]
    for a, b in zip(lens_q, lens_k):
        cq.append(cq[-1] + a)
        ck.append(ck[-1] + b)
    max_k = max(lens_k)
    g = torch.Generator(device="cpu").manual_seed(3)
    inp = torch.randn(2, cq[-1], max_k, generator=g).to(dtype)
    args = dict(local_blocks=3, init_blocks=2, block_size=64, stride=16, clip=clip)
    t = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)  # noqa: E731
    got = max_pooling_1d_varlen(inp.to(DEV), t(cq), t(ck), t(cache), max(lens_q), max_k,
                                **args).cpu()
    want = oracle.page_maxpool_varlen(inp, cq, ck, cache, max(lens_q), max_k, **args)
    assert got.shape == want.shape
    assert torch.equal(got.double(), want.double())
    other = oracle.page_maxpool_varlen(inp, cq, ck, cache, max(lens_q), max_k,
                                       **{**args, "clip": "row" if clip == "sequence" else "sequence"})
    assert not torch.equal(got.double(), other.double())
    buf = torch.empty_like(got, device=DEV)
    got2 = max_pooling_1d_varlen(inp.to(DEV), t(cq), t(ck), t(cache), max(lens_q), max_k,
                                 buf=buf, **args)
    assert got2.data_ptr() == buf.data_ptr() and torch.equal(got2.cpu(), got)


# ---------------------------------------------------------------------------
# Fused two-stage selection
# ---------------------------------------------------------------------------
def _nosa_select(case, cis, **kw):
    kc, cu_c = compress_k(case.k, case.cu_seqlens, cu_seqlens_host=case.cu_host)
    ids = nosa_prefill_topk_idx(case.q, kc, cis.to(DEV), case.cu_seqlens, cu_c, case.cu_seqlens,
                                case.selector, cu_seqlens_q_host=case.cu_host, **kw)
    return kc, cu_c, ids


def _gpu_page_scores(case, kc, cu_c_host, rows, out_len):
    """The GPU's qk page scores (no forcing) of the given rows, [G, R, out_len]."""
    G = kc.shape[1]
    res = torch.full((G, len(rows), out_len), float("-inf"), dtype=torch.float64)
    cu = case.cu_host
    for b in range(len(cu) - 1):
        sel = [i for i, r in enumerate(rows) if cu[b] <= r < cu[b + 1]]
        a0, a1 = cu_c_host[b], cu_c_host[b + 1]
        if not sel or a1 <= a0:
            continue
        n = cu[b + 1] - cu[b]
        sc = case.selector.score_pages(case.q[cu[b] : cu[b + 1]], kc[a0:a1], seq_len=n,
                                       block_size=64, kernel_stride=16).cpu().double()
        loc = torch.tensor([rows[i] - cu[b] for i in sel])
        w = min(out_len, sc.shape[-1])
        res[:, torch.tensor(sel), :w] = sc[:, loc, :w]
    return res


def _check_nosa_select(case, cis, rows, *, topk, init, local, select, max_band_rows=0,
                       clip="sequence"):
    kc, cu_c, ids = _nosa_select(case, cis, topk=topk, init_blocks=init, local_blocks=local,
                                 select_blocks=select, pool_clip=clip)
    cu = case.cu_host
    max_q = case.max_seqlen
    out_len = (max_q + 63) // 64
    G, total, take = ids.shape
    assert take == min(topk, out_len)
    got = ids.cpu()[:, rows]
    cu_c_host = cu_c.cpu().tolist()
    q_idx = oracle.nosa_q_idx(cu, max_q)[torch.tensor(rows)]
    # (1) bit-exact against the oracle's selection on the GPU's intermediates.
    page_qk = _gpu_page_scores(case, kc, cu_c_host, rows, out_len)
    means = nosa_mean_pooling(cis.to(DEV), case.cu_seqlens, max_q).cpu()
    block, block_cis = oracle.nosa_pool_rows(page_qk, means, cu, cu_c_host, rows,
                                             out_len=out_len, init_blocks=init,
                                             local_blocks=local, clip=clip)
    want_same = oracle.nosa_two_stage(block, block_cis, q_idx, topk=topk,
                                      qk_select=init + local + select)
    diff = (got != want_same).any(-1)
    assert not bool(diff.any()), f"rows {diff.nonzero()[:5].tolist()} differ from the oracle tail"
    # (2) against the independent oracle (its own scores), on the GPU's compressed keys.
    qf, kf = oracle.fused_weights(case.selector.head_mix.cpu(), case.selector.kv_head_mix.cpu(),
                                  case.selector.q_proj.cpu(), case.selector.k_proj.cpu(),
                                  case.q.dtype)
    atom = oracle.nosa_atom_scores(case.q.cpu(), kc.cpu(), cu, cu_c_host, qf, kf, rows=rows)
    want, blk, over = oracle.nosa_select_prefill(
        atom, cis, cu, cu_c_host, cu, max_q, max_q, topk=topk, init_blocks=init,
        local_blocks=local, select_blocks=select, rows=rows, return_scores=True, clip=clip)
    rep = oracle.check_nosa_topk(got, want, blk, over, topk=topk, qk_select=init + local + select)
    print(f"\nNOSA selection vs independent oracle: {rep}")
    assert rep.ok, str(rep)
    assert rep.band_rows <= max_band_rows, str(rep)
    return ids


def test_nosa_select_10k_paper_budget():
    """topk 96 = 1 sink + 16 local + 79 CIS-ranked, shortlist 41 (the NOSA defaults)."""
    case = workloads.hidden_space_layer((10000,), device=DEV, seed=11)
    cis = _cis(10000, 2, seed=11)
    rows = spread_rows(case.cu_host, per_seq=96)
    _check_nosa_select(case, cis, rows, topk=96, init=1, local=16, select=24)


@pytest.mark.parametrize("clip", ["sequence", "row"])
def test_nosa_select_ragged_q_idx_alignment(clip):
    """Shorter sequences' q_idx is right-aligned to the longest one: their late
    pages pass the q_idx mask, and -1 fills the ids past it.  Under the row
    clip those late pages pool the CIS means' zero padding (score 0, above
    about half of the real pages), so the two clips choose different pages."""
    lens = (3000, 700, 31, 4500, 64)
    case = workloads.hidden_space_layer(lens, device=DEV, seed=12)
    cis = _cis(sum(lens), 2, seed=12)
    rows = spread_rows(case.cu_host, per_seq=64)
    ids = _check_nosa_select(case, cis, rows, topk=12, init=1, local=2, select=3, clip=clip)
    assert ids.shape == (2, sum(lens), 12)
    if clip == "row":
        _, _, seq_ids = _nosa_select(case, cis, topk=12, init_blocks=1, local_blocks=2,
                                     select_blocks=3)
        assert not torch.equal(ids.cpu(), seq_ids.cpu())


def test_nosa_select_with_nan_and_inf_scores():
    """NaN and infinities in the qk scores.  NOSA's selection has no -1 rule for
    them (nosa.py:1288-1305: only ids past q_idx become -1): ``torch.topk``
    ranks NaN above +inf, so NaN pages enter the shortlist first (ties to the
    lower page) and are then chosen at +inf in stage 2.  Planted in query rows
    (every page of the row's group scores NaN, or mixes +-inf) and in key rows
    (the pages around one window score NaN for every row)."""
    import dataclasses
    case = workloads.hidden_space_layer((6000,), device=DEV, seed=16)
    q, k = case.q.clone(), case.k.clone()
    nan, inf = float("nan"), float("inf")
    for r, h, d, val in ((700, 3, 5, nan), (2600, 20, 9, nan), (4100, 5, 77, inf),
                         (5100, 21, 3, -inf)):
        q[r, h, d] = val
    k[64 * 30 + 7, 1, 9] = nan
    k[64 * 50 + 2, 0, 4] = inf
    case = dataclasses.replace(case, q=q, k=k)
    cis = _cis(6000, 2, seed=16)
    rows = sorted(set(spread_rows(case.cu_host, per_seq=64)) | {700, 2600, 4100, 5100, 64 * 31,
                                                                64 * 51 + 3})
    _check_nosa_select(case, cis, rows, topk=24, init=1, local=4, select=6)


def test_nosa_select_long_rows_fast_and_general_paths():
    """Rows of more than 256 pages: bf16 stage 1 takes a fast path while its
    shortlist bound is a positive score and no score is NaN or +inf, else the
    general path.  Keys shifted along one direction make most of a row's scores
    share the sign of q~ . shift (both paths occur), a zero query row ties every
    page at +0, and a NaN query row scores NaN everywhere."""
    import dataclasses
    case = workloads.hidden_space_layer((20000,), hidden=1024, device=DEV, seed=17)
    gen = torch.Generator(device="cpu").manual_seed(6)
    shift = (torch.randn(case.k.shape[1:], generator=gen) * 20.0).to(DEV)
    k = (case.k.float() + shift).to(case.k.dtype)
    q = case.q.clone()
    q[[15000, 19999]] = 0
    q[17000, 3, 5] = float("nan")
    case = dataclasses.replace(case, q=q, k=k)
    cis = _cis(20000, 2, seed=17)
    rows = sorted(set(spread_rows(case.cu_host, per_seq=64)) | {15000, 17000, 19999})
    _check_nosa_select(case, cis, rows, topk=96, init=1, local=16, select=24)


def test_nosa_select_long_rows_of_tied_scores():
    """Every key row equal: every page of a row ties in stage 1, so rows with a
    positive score gather more than 256 ties and leave the fast path, and the
    shortlist takes the lowest pages."""
    import dataclasses
    case = workloads.hidden_space_layer((20000,), hidden=1024, device=DEV, seed=18)
    case = dataclasses.replace(case, k=case.k[:1].expand_as(case.k).contiguous())
    cis = _cis(20000, 2, seed=18)
    rows = spread_rows(case.cu_host, per_seq=48)
    _check_nosa_select(case, cis, rows, topk=96, init=1, local=16, select=24)


def test_nosa_select_fp32_and_fp16():
    case = workloads.head_space_layer(5000, device=DEV, seed=13)
    cis = _cis(5000, 2, torch.float32, seed=13)
    rows = spread_rows(case.cu_host, per_seq=96)
    _check_nosa_select(case, cis, rows, topk=20, init=2, local=3, select=6)
    case = workloads.hidden_space_layer((6000,), device=DEV, dtype=torch.float16, seed=14)
    cis = _cis(6000, 2, torch.float16, seed=14)
    rows = spread_rows(case.cu_host, per_seq=64)
    _check_nosa_select(case, cis, rows, topk=40, init=1, local=8, select=10)


def test_nosa_select_tied_cis_scores():
    """Constant CIS (every page ties in stage 2): the lower pages win."""
    case = workloads.hidden_space_layer((4000,), device=DEV, seed=15)
    cis = torch.zeros(4000, 2, dtype=torch.bfloat16)
    rows = spread_rows(case.cu_host, per_seq=64)
    _check_nosa_select(case, cis, rows, topk=16, init=1, local=2, select=4)


# ---------------------------------------------------------------------------
# CIS-biased attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("clip", ["sequence", "row"])
def test_nosa_select_batch_without_any_compressed_key(clip):
    """No compressed key in the whole batch: the plans are the forced pages only."""
    lens = (20, 3, 31)
    case = workloads.hidden_space_layer(lens, device=DEV, seed=21)
    cis = _cis(sum(lens), 2, seed=21)
    _check_nosa_select(case, cis, list(range(sum(lens))), topk=8, init=1, local=2, select=2,
                       clip=clip)


def _check_nosa_attention(case, cis, ids, rows, **kw):
    out, lse = nosa_sparse_attention(case.q, case.k, case.v, cis.to(DEV), case.cu_seqlens,
                                     case.cu_seqlens, case.max_seqlen, case.max_seqlen, ids,
                                     return_lse=True, **kw)
    want, want_lse = oracle.nosa_attention(case.q.cpu(), case.k.cpu(), case.v.cpu(), cis,
                                           case.cu_host, case.cu_host, ids.cpu()[:, rows],
                                           rows=rows, ids_rows_aligned=True, return_lse=True,
                                           **kw)
    ok, mx, mr = oracle.check_attention(out.cpu()[rows], want)
    print(f"\nNOSA attention parity: max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert ok, (mx, mr)
    got_lse = lse.cpu()[:, rows].double()
    fin = torch.isfinite(want_lse)
    assert torch.equal(torch.isfinite(got_lse), fin)
    torch.testing.assert_close(got_lse[fin], want_lse[fin], rtol=1e-4, atol=2e-3)
    return out


def test_nosa_attention_bf16():
    case = workloads.hidden_space_layer((3000,), device=DEV, seed=16)
    cis = _cis(3000, 2, seed=16)
    _, _, ids = _nosa_select(case, cis, topk=24, init_blocks=1, local_blocks=4, select_blocks=6)
    _check_nosa_attention(case, cis, ids, spread_rows(case.cu_host, per_seq=64))


def test_nosa_attention_fp16_scale_and_wide_cis():
    """CIS spread of several units (weights over e^+-12) exercises the rescaling."""
    case = workloads.hidden_space_layer((2500,), device=DEV, dtype=torch.float16, seed=17)
    cis = _cis(2500, 2, torch.float32, seed=17, std=4.0)
    _, _, ids = _nosa_select(case, cis, topk=24, init_blocks=1, local_blocks=4, select_blocks=6)
    _check_nosa_attention(case, cis, ids, spread_rows(case.cu_host, per_seq=48),
                          softmax_scale=0.05)


def test_nosa_attention_ragged_and_zero_bias_matches_plain():
    lens = (1, 31, 65, 700, 2000)
    case = workloads.hidden_space_layer(lens, device=DEV, seed=18)
    cis = _cis(sum(lens), 2, seed=18)
    _, _, ids = _nosa_select(case, cis, topk=16, init_blocks=1, local_blocks=2, select_blocks=4)
    rows = spread_rows(case.cu_host, per_seq=40)
    _check_nosa_attention(case, cis, ids, rows)
    # Sequences shorter than one compression window still get their forced
    # pages (the page max-pool overlays them whatever the scores).
    assert bool((ids[:, :32, 0] == 0).all())
    # A constant bias leaves the softmax unchanged.
    const = torch.full((sum(lens), 2), 0.75, dtype=torch.bfloat16, device=DEV)
    a = nosa_sparse_attention(case.q, case.k, case.v, const, case.cu_seqlens, case.cu_seqlens,
                              case.max_seqlen, case.max_seqlen, ids)
    b = sparse_attention(case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens,
                         case.max_seqlen, case.max_seqlen, ids)
    ok, mx, mr = oracle.check_attention(a.cpu(), b.cpu(), max_abs=1e-2, mean_rel=2e-3)
    assert ok, (mx, mr)


def test_nosa_prefill_end_to_end():
    case = workloads.hidden_space_layer((8000,), device=DEV, seed=19)
    cis = _cis(8000, 2, seed=19)
    out, ids = nosa_sparse_prefill(case.q, case.k, case.v, cis.to(DEV), case.cu_seqlens,
                                   case.selector, cu_seqlens_host=case.cu_host,
                                   return_topk_idx=True)
    assert ids.shape == (2, 8000, 96)
    rows = spread_rows(case.cu_host, per_seq=24)
    want = oracle.nosa_attention(case.q.cpu(), case.k.cpu(), case.v.cpu(), cis, case.cu_host,
                                 case.cu_host, ids.cpu()[:, rows], rows=rows,
                                 ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(out.cpu()[rows], want)
    assert ok, (mx, mr)
