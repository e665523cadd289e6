"""GPU parity at the benchmark configurations' full sizes, on sampled rows:

* the 128K MiniCPM4.1-8B attention layer (selection and attention, including
  the last query block and the attention tiles with the largest page unions);
* the ragged 8K+24K+48K+96K batch (per-sequence selection and attention);
* the whole 32-layer MiniCPM4.1-8B-shaped prefill at 64K (layer-0 stages
  against the oracle, then the full prefill finite and deterministic);
* the NOSA layer at 128K;
* attention paths the layer workloads do not reach: large V magnitudes (the
  per-page V exponent) and query sequences shorter than their key sequences.

Rows are sampled because the oracle is a float64 CPU loop; everything else
(plan invariants, determinism) is checked over the whole output.
"""
import pytest
import torch

import oracle
from gpu_helpers import oracle_select_rows, plan_structure_errors, spread_rows
from leanselect_amd import minicpm, workloads
from leanselect_amd.ops import (compress_k, leanselect_prefill_topk_idx, nosa_prefill_topk_idx,
                                nosa_sparse_attention, sparse_attention)
from leanselect_amd.ops.attention import attention_tile_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _select(case):
    kc, cu_c = compress_k(case.k, case.cu_seqlens, cu_seqlens_host=case.cu_host)
    ids = leanselect_prefill_topk_idx(
        case.q, kc, case.cu_seqlens, cu_c, case.selector, topk=case.topk,
        init_blocks=case.init_blocks, local_blocks=case.local_blocks,
        cu_seqlens_q_host=case.cu_host)
    return kc, cu_c, ids


def tile_unions(ids: torch.Tensor, cu_host: list[int], tile: int | None = None):
    """(group, first row, distinct pages) of every ``tile``-row tile of each sequence
    (by default the attention kernel's tile for this plan width)."""
    G, N, T = ids.shape
    tile = tile or attention_tile_rows(T)
    res = []
    for b in range(len(cu_host) - 1):
        s, e = cu_host[b], cu_host[b + 1]
        n = (e - s) // tile
        if n == 0:
            continue
        x = ids[:, s : s + n * tile].reshape(G, n, tile * T)
        xs = x.sort(-1).values
        first = torch.ones_like(xs[..., :1], dtype=torch.bool)
        distinct = (xs >= 0) & torch.cat([first, xs[..., 1:] != xs[..., :-1]], -1)
        u = distinct.sum(-1).cpu()
        for g in range(G):
            for i in range(n):
                res.append((g, s + i * tile, int(u[g, i])))
    return res


def widest_tile_rows(ids, cu_host, count=2, tile=None):
    """All rows of the ``count`` tiles with the largest unions (per group)."""
    tile = tile or attention_tile_rows(ids.shape[-1])
    un = tile_unions(ids, cu_host, tile)
    rows, best = set(), []
    for g in range(ids.shape[0]):
        cand = sorted((u for u in un if u[0] == g), key=lambda u: -u[2])[:count]
        best += cand
        for _, r0, _ in cand:
            rows.update(range(r0, r0 + tile))
    return sorted(rows), best


def _parity(case, ids, kc, cu_c, rows, *, check_select=True, require_exact=True,
            literal=False):
    if check_select:
        want_ids, scores = oracle_select_rows(case, kc.cpu(), cu_c.cpu().tolist(), rows,
                                              case.q.dtype)
        rep = oracle.check_topk(ids.cpu()[:, rows], want_ids, scores, case.q.dtype)
        print(f"\nselect parity: {rep}", flush=True)
        assert rep.ok, str(rep)
        if require_exact:
            assert rep.exact_rows == rep.rows and rep.band_rows == 0, str(rep)
    out = sparse_attention(case.q, case.k, case.v, case.cu_seqlens, case.cu_seqlens,
                           case.max_seqlen, case.max_seqlen, ids)
    want, _ = oracle.sparse_attention(case.q.cpu(), case.k.cpu(), case.v.cpu(), case.cu_host,
                                      case.cu_host, ids.cpu()[:, rows], rows=rows,
                                      ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(out.cpu()[rows], want, literal=literal)
    print(f"attention parity{' (literal 2e-2)' if literal else ''}: rows={len(rows)} "
          f"max_abs={mx:.3e} mean_rel={mr:.3e} max|out|={want.abs().max().item():.2f}", flush=True)
    assert ok, (mx, mr)
    return out


def test_layer_128k_unit_scale_literal_bound():
    """The headline layer at unit scale: each planted row gets one
    topic-amplitude vector however many blocks chose its page, and values have
    std about 0.5, so every output lies inside (-4, 4), where one bf16 step is
    at most 2^-6.  Selection exact and attention within the literal max-abs
    2e-2 and mean-relative 1e-3, with no quantisation-step allowance."""
    case = workloads.hidden_space_layer((131072,), device=DEV, seed=24, **workloads.UNIT_SCALE)
    kc, cu_c, ids = _select(case)
    assert not plan_structure_errors(ids, case.cu_host, 64, 1, 4)
    wide, best = widest_tile_rows(ids, case.cu_host)
    N = case.cu_host[-1]
    rows = sorted(set(spread_rows(case.cu_host, per_seq=48)) | set(wide) |
                  set(range(N - 64, N)))
    out = _parity(case, ids, kc, cu_c, rows, literal=True)
    assert float(out.abs().max()) < 4.0


def test_c1_layer_fp32_selection_bf16_attention():
    """The CPU-runnable layer (4096 tokens, 8q/2kv, GQA 4, budget 16 = 1 sink + 2
    local blocks): selection in float32, bit-exact on every row, and its plans
    through the bf16 attention kernel (the attention kernels, like the upstream
    ones, take fp16 and bf16 only) against the oracle on the same bf16 inputs."""
    case = workloads.head_space_layer(4096, device=DEV)
    kc, cu_c, ids = _select(case)
    assert ids.shape == (2, 4096, 16)
    assert not plan_structure_errors(ids, case.cu_host, 16, 1, 2)
    rows = list(range(4096))
    want_ids, scores = oracle_select_rows(case, kc.cpu(), cu_c.cpu().tolist(), rows, torch.float32)
    rep = oracle.check_topk(ids.cpu(), want_ids, scores, torch.float32)
    print(f"\nC1 select parity: {rep}", flush=True)
    assert rep.ok and rep.exact_rows == rep.rows, str(rep)
    q, k, v = (t.to(torch.bfloat16) for t in (case.q, case.k, case.v))
    out = sparse_attention(q, k, v, case.cu_seqlens, case.cu_seqlens, 4096, 4096, ids)
    arows = sorted(set(spread_rows(case.cu_host, per_seq=256)) | set(range(4096 - 64, 4096)))
    want, _ = oracle.sparse_attention(q.cpu(), k.cpu(), v.cpu(), case.cu_host, case.cu_host,
                                      ids.cpu()[:, arows], rows=arows, ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(out.cpu()[arows], want, literal=True)
    print(f"C1 attention parity (bf16, literal 2e-2): rows={len(arows)} max_abs={mx:.3e} "
          f"mean_rel={mr:.3e}", flush=True)
    assert ok, (mx, mr)


def test_layer_128k_selection_and_attention():
    """The headline layer: 131072 tokens, 32q/2kv, budget 64 (1 sink + 4 local blocks)."""
    case = workloads.hidden_space_layer((131072,), device=DEV, seed=21)
    kc, cu_c, ids = _select(case)
    assert not plan_structure_errors(ids, case.cu_host, 64, 1, 4)
    wide, best = widest_tile_rows(ids, case.cu_host)
    print(f"\nwidest tiles (group, first row, union pages): {best}", flush=True)
    assert all(u > 100 for _, _, u in best)
    N = case.cu_host[-1]
    rows = sorted(set(spread_rows(case.cu_host, per_seq=48)) | set(wide) |
                  set(range(N - 64, N)))
    _parity(case, ids, kc, cu_c, rows)


def test_layer_128k_fp16():
    """The headline layer's shapes in float16 (selection scored and attention run in
    fp16), on spread rows including the last block."""
    case = workloads.hidden_space_layer((131072,), device=DEV, seed=23, dtype=torch.float16)
    kc, cu_c, ids = _select(case)
    assert not plan_structure_errors(ids, case.cu_host, 64, 1, 4)
    N = case.cu_host[-1]
    rows = sorted(set(spread_rows(case.cu_host, per_seq=32)) | set(range(N - 32, N)))
    _parity(case, ids, kc, cu_c, rows)  # as measured: every sampled row exact


def test_ragged_8k_24k_48k_96k():
    """Four packed sequences: selection and attention stay inside each sequence."""
    case = workloads.hidden_space_layer((8192, 24576, 49152, 98304), device=DEV, seed=22)
    kc, cu_c, ids = _select(case)
    assert not plan_structure_errors(ids, case.cu_host, 64, 1, 4)
    wide, _ = widest_tile_rows(ids, case.cu_host, count=1)
    rows = sorted(set(spread_rows(case.cu_host, per_seq=24)) | set(wide))
    out = _parity(case, ids, kc, cu_c, rows)
    # Each sequence alone gives the same plans and outputs (no cross-sequence state).
    cu = case.cu_host
    for b in (0, 2):
        s, e = cu[b], cu[b + 1]
        one = workloads.LayerCase(
            q=case.q[s:e], k=case.k[s:e], v=case.v[s:e],
            cu_seqlens=torch.tensor([0, e - s], dtype=torch.int32, device=DEV),
            cu_host=[0, e - s], selector=case.selector, topk=case.topk,
            init_blocks=case.init_blocks, local_blocks=case.local_blocks)
        _, _, ids1 = _select(one)
        assert torch.equal(ids1, ids[:, s:e])
        out1 = sparse_attention(one.q, one.k, one.v, one.cu_seqlens, one.cu_seqlens, e - s, e - s,
                                ids1)
        assert torch.equal(out1, out[s:e])


def test_whole_model_prefill_64k():
    """The full MiniCPM4.1-8B-shaped model at 64K: layer 0 stage by stage on sampled
    rows (RoPE exact, plans, attention), then the 32-layer prefill twice."""
    cfg = minicpm.MiniCPMConfig()
    model = minicpm.MiniCPMLeanSelect(cfg, device=DEV, seed=31)
    N = 65536
    gen = torch.Generator(device=DEV).manual_seed(32)
    tok = torch.randint(0, cfg.vocab_size, (N,), generator=gen, device=DEV, dtype=torch.int32)
    cu_host = [0, N]
    cu = torch.tensor(cu_host, dtype=torch.int32, device=DEV)
    pos = model.positions(cu_host, DEV)
    H, G, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    with torch.no_grad():
        x = minicpm.embed_scale(tok, model.embed, cfg.scale_emb)
        h = minicpm.rms_layernorm(x, model.layers[0].input_norm, cfg.rms_norm_eps)
        rows = spread_rows(cu_host, per_seq=64)
        ridx = torch.tensor(rows, device=DEV)
        qkv_pre = torch.nn.functional.linear(h, model.layers[0].w_qkv)[ridx].cpu()
        o, parts = model.attention(0, h, pos, cu, cu_host, return_parts=True)
        torch.cuda.synchronize()
    cos, sin = model.rope_tables(N)
    qkv = parts["qkv"]
    got_q = qkv[ridx, : H * D].cpu().view(len(rows), H, D)
    want_q = oracle.apply_rotary_pos_emb(qkv_pre[:, : H * D].view(len(rows), H, D), cos.cpu(),
                                         sin.cpu(), torch.tensor(rows))
    assert torch.equal(got_q, want_q)
    q = qkv[:, : H * D].view(N, H, D).cpu()
    k = qkv[:, H * D : H * D + G * D].view(N, G, D).cpu()
    v = qkv[:, H * D + G * D :].view(N, G, D).cpu()
    sel = model.layers[0].selector
    kc, cu_c = oracle.compress_k(k, cu_host)
    qf, kf = oracle.fused_weights(sel.head_mix.cpu(), sel.kv_head_mix.cpu(), sel.q_proj.cpu(),
                                  sel.k_proj.cpu(), q.dtype)
    want_ids, scores = oracle.select_prefill(
        q, kc, cu_host, cu_c.tolist(), qf, kf, topk=cfg.topk, init_blocks=cfg.init_blocks,
        local_blocks=cfg.local_blocks, rows=rows, return_scores=True)
    got_ids = parts["topk_idx"].cpu()
    rep = oracle.check_topk(got_ids[:, rows], want_ids, scores, q.dtype)
    print(f"\nlayer-0 select parity: {rep}", flush=True)
    assert rep.ok and rep.band_rows == 0, str(rep)
    want, _ = oracle.sparse_attention(q, k, v, cu_host, cu_host, got_ids[:, rows], rows=rows,
                                      ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(parts["attn"].cpu()[rows], want)
    print(f"layer-0 attention parity: max_abs={mx:.3e} mean_rel={mr:.3e}", flush=True)
    assert ok, (mx, mr)
    del parts, qkv, o, h, x, q, k, v
    l1 = model.prefill(tok, cu_host)
    l2 = model.prefill(tok, cu_host)
    torch.cuda.synchronize()
    assert l1.shape == (1, cfg.vocab_size) and bool(torch.isfinite(l1).all())
    assert torch.equal(l1, l2)


def test_nosa_layer_128k():
    """NOSA at 128K (budget 96 = 1 sink + 16 local + 79 CIS-ranked, shortlist 41):
    gap-aware selection against the independent oracle, then attention."""
    case = workloads.hidden_space_layer((131072,), device=DEV, seed=23)
    g = torch.Generator(device="cpu").manual_seed(24)
    cis = torch.randn(131072, 2, generator=g).to(torch.bfloat16)
    kc, cu_c = compress_k(case.k, case.cu_seqlens, cu_seqlens_host=case.cu_host)
    topk, init, local, select = 96, 1, 16, 24
    ids = nosa_prefill_topk_idx(case.q, kc, cis.to(DEV), case.cu_seqlens, cu_c, case.cu_seqlens,
                                case.selector, topk=topk, init_blocks=init, local_blocks=local,
                                select_blocks=select, cu_seqlens_q_host=case.cu_host)
    N = case.cu_host[-1]
    rows = sorted(set(spread_rows(case.cu_host, per_seq=48)) | set(range(N - 16, N)))
    cu, cu_c_host = case.cu_host, cu_c.cpu().tolist()
    qf, kf = oracle.fused_weights(case.selector.head_mix.cpu(), case.selector.kv_head_mix.cpu(),
                                  case.selector.q_proj.cpu(), case.selector.k_proj.cpu(),
                                  case.q.dtype)
    atom = oracle.nosa_atom_scores(case.q.cpu(), kc.cpu(), cu, cu_c_host, qf, kf, rows=rows)
    want, blk, over = oracle.nosa_select_prefill(
        atom, cis, cu, cu_c_host, cu, N, N, topk=topk, init_blocks=init, local_blocks=local,
        select_blocks=select, rows=rows, return_scores=True)
    rep = oracle.check_nosa_topk(ids.cpu()[:, rows], want, blk, over, topk=topk,
                                 qk_select=init + local + select)
    print(f"\nNOSA 128K selection: {rep}", flush=True)
    assert rep.ok and rep.band_rows == 0, str(rep)
    out = nosa_sparse_attention(case.q, case.k, case.v, cis.to(DEV), case.cu_seqlens,
                                case.cu_seqlens, N, N, ids)
    want_o = oracle.nosa_attention(case.q.cpu(), case.k.cpu(), case.v.cpu(), cis, cu, cu,
                                   ids.cpu()[:, rows], rows=rows, ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(out.cpu()[rows], want_o)
    print(f"NOSA 128K attention: max_abs={mx:.3e} mean_rel={mr:.3e}", flush=True)
    assert ok, (mx, mr)


def test_attention_large_v_page_exponents():
    """Pages whose V exceeds fp16's range (|V| ~ 1e5 and ~ 1e7): the staged V^T
    carries a per-page power-of-two exponent, and exponents above 7 force the
    rescale path.  With values this large an output element can be a small
    difference of huge terms, so each element's error is bounded relative to
    the magnitude it is summed from, sum_j p_j |v_j|: 2^-10 of it covers the
    11-bit (fp16) weights of the P.V product plus the output's rounding (a
    bf16 P, as the reference's kernel uses, would need 2^-7)."""
    case = workloads.hidden_space_layer((4096,), device=DEV, seed=25)
    _, _, ids = _select(case)
    v = case.v.clone()
    for p, scale in ((0, 1e5), (3, 1e7), (17, 3e4), (40, 2e6)):
        v[64 * p : 64 * p + 64] = (v[64 * p : 64 * p + 64].float() * scale).to(v.dtype)
    assert float(v.float().abs().max()) > 32768 * 128
    out = sparse_attention(case.q, case.k, v, case.cu_seqlens, case.cu_seqlens, 4096, 4096, ids)
    rows = spread_rows(case.cu_host, per_seq=64)
    want, _, mass = oracle.sparse_attention(case.q.cpu(), case.k.cpu(), v.cpu(), case.cu_host,
                                            case.cu_host, ids.cpu()[:, rows], rows=rows,
                                            ids_rows_aligned=True, return_abs=True)
    got = out.cpu()[rows].double()
    b = want.double()
    err = (got - b).abs()
    bound = 2.0 ** -10 * mass + oracle.output_step(b, torch.bfloat16)
    worst = float((err / bound).max())
    mr = float(err.mean() / b.abs().mean())
    print(f"\nlarge-V attention: worst error / bound = {worst:.3f} mean_rel={mr:.3e}", flush=True)
    assert worst <= 1.0 and mr <= 1e-3
    assert bool(torch.isfinite(out).all())


def test_attention_queries_shorter_than_keys():
    """len_q < len_k per sequence under causal=True: row t of a sequence sees keys
    j <= t + len_k - len_q (the queries are the last len_q positions)."""
    lens_q, lens_k = (100, 700, 1500, 1), (300, 700, 2600, 65)
    cq, ck = [0], [0]
    for a, b in zip(lens_q, lens_k):
        cq.append(cq[-1] + a)
        ck.append(ck[-1] + b)
    g = torch.Generator(device="cpu").manual_seed(26)
    H, G, D, T = 32, 2, 128, 24
    q = torch.randn(cq[-1], H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(ck[-1], G, D, generator=g).to(torch.bfloat16)
    v = torch.randn(ck[-1], G, D, generator=g).to(torch.bfloat16)
    ids = torch.full((G, cq[-1], T), -1, dtype=torch.int32)
    for b in range(len(lens_q)):
        for t in range(lens_q[b]):
            last = (t + lens_k[b] - lens_q[b]) // 64  # the row's last visible page
            for gg in range(G):
                pages = torch.randperm(last + 1, generator=g)[: min(T - 2, last + 1)]
                ids[gg, cq[b] + t, : pages.numel()] = pages.to(torch.int32)
    ids[:, :, -1] = 10_000  # out of range: ignored
    t32 = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)  # noqa: E731
    out = sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), t32(cq), t32(ck), max(lens_q),
                           max(lens_k), ids.to(DEV))
    rows = sorted(set(spread_rows(cq, per_seq=40)))
    want, _ = oracle.sparse_attention(q, k, v, cq, ck, ids[:, rows], rows=rows,
                                      ids_rows_aligned=True)
    ok, mx, mr = oracle.check_attention(out.cpu()[rows], want)
    print(f"\nlen_q < len_k attention: max_abs={mx:.3e} mean_rel={mr:.3e}", flush=True)
    assert ok, (mx, mr)
