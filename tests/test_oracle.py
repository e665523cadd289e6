"""Pins the CPU oracle against the reference's known answers, closed forms and
brute force (no GPU).  Reference citations are paths in the LeanSelect repo."""
import json
import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

import oracle
from leanselect_amd.selector import LeanSelectSelector

GOLDEN = Path(__file__).with_name("golden")


# --------------------------------------------------------------------------
# Page pooling
# --------------------------------------------------------------------------
def test_pool_matches_reference_known_answers():
    data = json.loads((GOLDEN / "pool_pages.json").read_text())
    c0, c1 = data["cases"]
    got = oracle.pool_atoms_to_pages(torch.tensor(c0["atoms"], dtype=torch.float32),
                                     seq_len=c0["seq_len"])
    assert got.tolist() == c0["expected"]
    got = oracle.pool_atoms_to_pages(torch.tensor(c1["atoms"]), seq_len=c1["seq_len"])
    assert got.nonzero().flatten().tolist() == c1["expected_nonzero_pages"]


@pytest.mark.parametrize("n_atoms,seq_len", [(1, 64), (3, 64), (15, 256), (31, 512), (30, 700),
                                             (200, 3000), (7, 1000)])
def test_pool_matches_padded_max_pool1d(n_atoms, seq_len):
    # Library routine: pad one -inf atom on the left (and on the right up to the
    # last window), then max_pool1d with kernel 5 and stride 4.
    x = torch.randn(3, n_atoms)
    n_pages = (seq_len + 63) // 64
    right = max((n_pages - 1) * 4 + 5 - (n_atoms + 1), 0)
    padded = F.pad(x[:, None], (1, right), value=float("-inf"))
    want = F.max_pool1d(padded, kernel_size=5, stride=4)[:, 0, :n_pages]
    got = oracle.pool_atoms_to_pages(x, seq_len=seq_len)
    assert torch.equal(got, want)


def test_pool_rejects_bad_geometry():
    with pytest.raises(ValueError):
        oracle.pool_atoms_to_pages(torch.ones(3), seq_len=64, kernel_stride=0)
    with pytest.raises(ValueError):
        oracle.pool_atoms_to_pages(torch.ones(3), seq_len=64, block_size=60)


# --------------------------------------------------------------------------
# Folded projections
# --------------------------------------------------------------------------
def _small_selector(seed=7, H=8, G=2, D=8, R=2, RD=4):
    torch.manual_seed(seed)
    sel = LeanSelectSelector(num_heads=H, num_kv_heads=G, head_dim=D, router_heads=R, router_dim=RD)
    with torch.no_grad():
        sel.head_mix.normal_()
        sel.kv_head_mix.normal_()
    return sel


def test_fold_matches_explicit_routes():
    # Restates the identity of tests/test_core.py:34-56 with an explicit loop
    # over routes and heads, in float64.
    sel = _small_selector()
    query = torch.randn(3, 8, 8, dtype=torch.float64)
    keys = torch.randn(7, 2, 8, dtype=torch.float64)
    qf, kf = oracle.fused_weights(sel.head_mix, sel.kv_head_mix, sel.q_proj, sel.k_proj,
                                  torch.float64)
    got = oracle.atom_scores(oracle.project_queries(query, qf, 2),
                             oracle.project_atom_keys(keys, kf))
    hm, khm = sel.head_mix.double(), sel.kv_head_mix.double()
    qp, kp = sel.q_proj.double(), sel.k_proj.double()
    want = torch.zeros(2, 3, 7, dtype=torch.float64)
    for g in range(2):
        for r in range(2):
            mixed = sum(query[:, h] * hm[h, r] for h in range(g * 4, (g + 1) * 4))
            want[g] += (mixed @ qp[r]) @ ((keys[:, g] * khm[g, r]) @ kp[r]).T
    # The fused weights are float32 products (selector.py:149-154), hence the
    # float32-level tolerance.
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)


def test_full_width_init_is_scaled_group_mean_dot():
    # tests/test_core.py:59-65: with R*F == D the initial router scores are
    # the group-mean query dot the key over sqrt(D).
    torch.manual_seed(7)
    sel = LeanSelectSelector(num_heads=8, num_kv_heads=2, head_dim=8, router_heads=2, router_dim=4)
    query, keys = torch.randn(3, 8, 8), torch.randn(7, 2, 8)
    qf, kf = oracle.fused_weights(sel.head_mix, sel.kv_head_mix, sel.q_proj, sel.k_proj,
                                  torch.float32)
    got = oracle.atom_scores(oracle.project_queries(query, qf, 2), oracle.project_atom_keys(keys, kf))
    want = torch.einsum("ngd,agd->gna", query.reshape(3, 2, 4, 8).mean(2), keys) / math.sqrt(8)
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-5)


def test_bf16_rounding_order_is_one_rounding_per_stage():
    sel = _small_selector(H=32, G=2, D=128, R=4, RD=32)
    q = torch.randn(16, 32, 128).to(torch.bfloat16)
    qf, _ = oracle.fused_weights(sel.head_mix, sel.kv_head_mix, sel.q_proj, sel.k_proj,
                                 torch.bfloat16)
    # The fused weights are one float32 product each, then rounded.
    want_qf = (sel.head_mix[:, None, :, None] * sel.q_proj.permute(1, 0, 2)[None]).reshape(32, 128, 128)
    assert torch.equal(qf, want_qf.to(torch.bfloat16))
    got = oracle.project_queries(q, qf, 2)
    exact = torch.einsum("ngsd,gsdf->gnf", q.double().reshape(16, 2, 16, 128),
                         qf.double().reshape(2, 16, 128, 128))
    assert got.dtype == torch.bfloat16
    assert (got.float() - exact).abs().max() <= (exact.abs() * 2 ** -8).max() + 1e-6


# --------------------------------------------------------------------------
# Compressed keys
# --------------------------------------------------------------------------
def test_compress_k_is_window_mean_per_sequence():
    lens = [100, 31, 32, 48, 0, 77]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    k = torch.randn(cu[-1], 2, 16, dtype=torch.float64)
    kc, cu_c = oracle.compress_k(k, cu)
    rows = []
    counts = []
    for b, n in enumerate(lens):
        m = (n - 32) // 16 + 1 if n >= 32 else 0
        counts.append(m)
        for a in range(m):
            rows.append(k[cu[b] + 16 * a : cu[b] + 16 * a + 32].mean(0))
    assert cu_c.tolist() == [0] + list(torch.tensor(counts).cumsum(0).tolist())
    torch.testing.assert_close(kc, torch.stack(rows), rtol=1e-14, atol=1e-14)


def test_compress_keys_mean_short_sequence_is_whole_mean():
    k = torch.randn(2, 20, 2, 8, dtype=torch.float64)
    got = oracle.compress_keys_mean(k)
    torch.testing.assert_close(got, k.mean(1, keepdim=True))
    k = torch.randn(1, 80, 2, 8, dtype=torch.float64)
    got = oracle.compress_keys_mean(k)
    assert got.shape == (1, 4, 2, 8)
    torch.testing.assert_close(got[0, 3], k[0, 48:80].mean(0))


# --------------------------------------------------------------------------
# Selection
# --------------------------------------------------------------------------
def _brute_select(q, kc, cu, cu_c, qf, kf, topk, init, local, dtype):
    """Per-token loops: rounded dots, 5-atom max, forcing, sort by (-score, page)."""
    G = kf.shape[0]
    H = q.shape[1]
    gs = H // G
    take = min(topk, max((cu[b + 1] - cu[b] + 63) // 64 for b in range(len(cu) - 1)))
    out = torch.full((G, cu[-1], take), -1, dtype=torch.int32)
    rnd = lambda x: torch.tensor(x, dtype=torch.float64).to(torch.float32).to(dtype).double().item()
    for b in range(len(cu) - 1):
        n, A = cu[b + 1] - cu[b], cu_c[b + 1] - cu_c[b]
        if n <= 0 or A <= 0:
            continue
        n_pages = (n + 63) // 64
        for g in range(G):
            kt = [[rnd(sum(float(kc[cu_c[b] + a, g, d]) * float(kf[g, d, f]) for d in range(kf.shape[1])))
                   for f in range(kf.shape[2])] for a in range(A)]
            for t in range(n):
                qt = [rnd(sum(float(q[cu[b] + t, g * gs + s, d]) * float(qf[g * gs + s, d, f])
                              for s in range(gs) for d in range(q.shape[2])))
                      for f in range(qf.shape[2])]
                atom = [rnd(sum(x * y for x, y in zip(qt, kt[a]))) for a in range(A)]
                qp = t // 64
                scored = []
                for p in range(n_pages):
                    window = [atom[a] for a in range(4 * p - 1, 4 * p + 4) if 0 <= a < A]
                    s = max(window) if window else -math.inf
                    if p > qp:
                        s = -math.inf
                    elif p < init or p + local >= qp:
                        s = math.inf
                    scored.append((s, p))
                chosen = sorted(scored, key=lambda x: (-x[0], x[1]))[: min(take, n_pages)]
                ids = sorted(p for s, p in chosen if s != -math.inf)
                out[g, cu[b] + t, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_select_matches_brute_force(dtype):
    torch.manual_seed(3)
    H, G, D, R, RD = 4, 2, 8, 2, 4
    sel = _small_selector(H=H, G=G, D=D, R=R, RD=RD)
    lens = [200, 40, 130]
    cu = [0, 200, 240, 370]
    q = torch.randn(cu[-1], H, D).to(dtype)
    k = torch.randn(cu[-1], G, D).to(dtype)
    kc, cu_c = oracle.compress_k(k, cu)
    qf, kf = oracle.fused_weights(sel.head_mix, sel.kv_head_mix, sel.q_proj, sel.k_proj, dtype)
    got = oracle.select_prefill(q, kc, cu, cu_c.tolist(), qf, kf, topk=3, init_blocks=1,
                                local_blocks=1)
    want = _brute_select(q, kc, cu, cu_c.tolist(), qf, kf, 3, 1, 1, dtype)
    assert torch.equal(got, want)


def test_select_invariants_match_reference_runtime_test():
    # tests/test_runtime.py:71-94: 256 queries, 15 atoms, topk 2 + window 64.
    torch.manual_seed(0)
    sel = LeanSelectSelector(num_heads=4, num_kv_heads=2, head_dim=16, router_heads=2, router_dim=8)
    queries, keys = torch.randn(256, 4, 16), torch.randn(15, 2, 16)
    qf, kf = oracle.fused_weights(sel.head_mix, sel.kv_head_mix, sel.q_proj, sel.k_proj, torch.float32)
    ids = oracle.select_prefill(queries, keys, [0, 256], [0, 15], qf, kf, topk=2 + 1,
                                init_blocks=1, local_blocks=1)
    visible = torch.arange(256)[None, :, None] // 64
    assert ids.dtype == torch.int32
    assert torch.all((ids < 0) | (ids <= visible))
    assert torch.all((ids == 0).any(-1))


def test_packed_selection_equals_independent_sequences():
    torch.manual_seed(5)
    sel = _small_selector(H=4, G=2, D=8, R=2, RD=4)
    lens = [300, 17, 129, 64]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    q = torch.randn(cu[-1], 4, 8)
    k = torch.randn(cu[-1], 2, 8)
    qf, kf = oracle.fused_weights(sel.head_mix, sel.kv_head_mix, sel.q_proj, sel.k_proj, torch.float32)
    kc, cu_c = oracle.compress_k(k, cu)
    packed = oracle.select_prefill(q, kc, cu, cu_c.tolist(), qf, kf, topk=4, init_blocks=1, local_blocks=1)
    take = packed.shape[-1]
    for b, n in enumerate(lens):
        kcb, cub = oracle.compress_k(k[cu[b] : cu[b + 1]], [0, n])
        one = oracle.select_prefill(q[cu[b] : cu[b + 1]], kcb, [0, n], cub.tolist(), qf, kf,
                                    topk=4, init_blocks=1, local_blocks=1)
        part = packed[:, cu[b] : cu[b + 1], : one.shape[-1]]
        assert torch.equal(part, one)
        assert torch.all(packed[:, cu[b] : cu[b + 1], one.shape[-1] : take] == -1)
    # The 17-token sequence has no compressed key, so its rows stay -1.
    assert torch.all(packed[:, cu[1] : cu[2]] == -1)


# --------------------------------------------------------------------------
# Sparse attention
# --------------------------------------------------------------------------
def _dense_masked(q, k, v, mask, scale):
    H, G = q.shape[1], k.shape[1]
    kk = k.repeat_interleave(H // G, dim=1).transpose(0, 1)
    vv = v.repeat_interleave(H // G, dim=1).transpose(0, 1)
    return F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv, attn_mask=mask,
                                          scale=scale).transpose(0, 1)


def test_sparse_attention_matches_dense_sdpa_with_page_mask():
    torch.manual_seed(11)
    N, H, G, D = 300, 4, 2, 16
    q = torch.randn(N, H, D, dtype=torch.float64)
    k = torch.randn(N, G, D, dtype=torch.float64)
    v = torch.randn(N, G, D, dtype=torch.float64)
    n_pages = (N + 63) // 64
    ids = torch.full((G, N, 3), -1, dtype=torch.int32)
    mask = torch.zeros(H, N, N, dtype=torch.bool)
    for t in range(N):
        for g in range(G):
            pages = torch.randperm(t // 64 + 1)[:3].tolist()
            pages.append(t // 64)  # duplicates must count once
            ids[g, t, : min(3, len(pages))] = torch.tensor(pages[:3], dtype=torch.int32)
            if len(pages) > 3:
                ids[g, t, 0] = t // 64
            sel = {p for p in ids[g, t].tolist() if p >= 0}
            for h in range(g * 2, g * 2 + 2):
                for p in sel:
                    mask[h, t, p * 64 : min(N, p * 64 + 64)] = True
            mask[g * 2 : g * 2 + 2, t, t + 1 :] = False
    out, lse = oracle.sparse_attention(q, k, v, [0, N], [0, N], ids)
    want = _dense_masked(q, k, v, mask, D ** -0.5)
    torch.testing.assert_close(out, want, rtol=1e-10, atol=1e-10)
    assert lse.shape == (H, N)
    assert n_pages == 5


def test_all_pages_selected_equals_causal_attention():
    torch.manual_seed(2)
    N, H, G, D = 200, 4, 1, 8
    q, k, v = (torch.randn(N, h, D, dtype=torch.float64) for h in (H, G, G))
    ids = torch.arange(4, dtype=torch.int32).repeat(G, N, 1)
    out, _ = oracle.sparse_attention(q, k, v, [0, N], [0, N], ids)
    want = _dense_masked(q, k, v, torch.ones(N, N, dtype=torch.bool).tril()[None], D ** -0.5)
    torch.testing.assert_close(out, want, rtol=1e-10, atol=1e-10)


def test_empty_row_gives_zero_and_inf_lse():
    q, k, v = torch.randn(5, 2, 8), torch.randn(5, 1, 8), torch.randn(5, 1, 8)
    ids = torch.full((1, 5, 2), -1, dtype=torch.int32)
    out, lse = oracle.sparse_attention(q, k, v, [0, 5], [0, 5], ids)
    assert torch.all(out == 0) and torch.all(torch.isinf(lse))


# --------------------------------------------------------------------------
# Parity rule
# --------------------------------------------------------------------------
def test_topk_checker_detects_planted_mistakes():
    scores = torch.tensor([[[math.inf, 5.0, 1.0, 4.0, 4.0 * (1 + 2 ** -9), 0.5, math.inf,
                             -math.inf]]], dtype=torch.float64)
    # take 4: forced {0, 6} + top-2 of {1: 5, 2: 1, 3: 4, 4: 4.0078, 5: .5}
    oracle_ids = torch.tensor([[[0, 1, 4, 6]]], dtype=torch.int32)
    rep = oracle.check_topk(oracle_ids, oracle_ids, scores, torch.float32)
    assert rep.exact_rows == 1 and rep.band_rows == 0
    # Pages 3 and 4 differ by 2**-9 relative, above the 1e-3 rule: a swap is a
    # failure in every dtype (one bf16 step is no excuse).
    swap = torch.tensor([[[0, 1, 3, 6]]], dtype=torch.int32)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        assert not oracle.check_topk(swap, oracle_ids, scores, dt).ok
    # An exact tie at the boundary may go either way (counted as a band row).
    tie = scores.clone()
    tie[0, 0, 4] = 4.0
    want = torch.tensor([[[0, 1, 3, 6]]], dtype=torch.int32)  # ties to the lower page
    rep = oracle.check_topk(torch.tensor([[[0, 1, 4, 6]]], dtype=torch.int32), want, tie,
                            torch.bfloat16)
    assert rep.ok and rep.band_rows == 1 and rep.exact_rows == 0
    # A near-tie inside 1e-3 relative is in the band too.
    near = scores.clone()
    near[0, 0, 4] = 4.0 * (1 + 5e-4)
    assert oracle.check_topk(swap, oracle_ids, near, torch.float32).ok
    # A page far below the boundary, a missing forced page, an invisible page.
    for bad in ([0, 1, 2, 6], [0, 1, 3, 4], [0, 1, 4, 7], [0, 1, 1, 6]):
        rep = oracle.check_topk(torch.tensor([[bad]], dtype=torch.int32), oracle_ids, scores,
                                torch.bfloat16)
        assert not rep.ok, bad


def test_attention_checker_tolerances():
    ref = torch.randn(64, 4, 128)
    ok, mx, mr = oracle.check_attention(ref + 1e-4, ref)
    assert ok and abs(mx - 1e-4) < 1e-6
    ok, _, _ = oracle.check_attention(ref + 3e-2, ref)
    assert not ok
    # The raw 2e-2 bound applies wherever the output dtype resolves it ...
    small = torch.full((1000,), 1.5)
    off = small.clone()
    off[0] += 0.03
    assert not oracle.check_attention(off.to(torch.bfloat16), small)[0]
    # ... and one bf16 step where a step is coarser (0.0625 at |x| = 10): two
    # correct roundings can land on neighbouring values there; two steps cannot.
    ref = torch.full((1000,), 10.0)
    one = ref.clone()
    one[0] += 0.0625
    ok, mx, _ = oracle.check_attention(one.to(torch.bfloat16), ref)
    assert ok and abs(mx - 0.0625) < 1e-9
    two = ref.clone()
    two[0] += 0.125
    assert not oracle.check_attention(two.to(torch.bfloat16), ref)[0]
    # float32 outputs get no step allowance.
    assert not oracle.check_attention(one, ref)[0]
    # The mean bound: a uniform 2e-3 relative offset fails it.
    assert not oracle.check_attention(ref * (1 + 2e-3), ref)[0]


def test_output_step_matches_the_formats():
    # Brute force through the format: the step at a representable x is the gap
    # to the next representable value (the bit pattern plus one).
    for dt in (torch.bfloat16, torch.float16):
        x = torch.tensor([0.3, 1.0, 1.5, 3.9, 4.0, 10.0, -6.0]).to(dt)
        bits = x.abs().view(torch.int16) + 1
        gap = bits.view(dt).double() - x.abs().double()
        assert torch.equal(oracle.output_step(x.double(), dt), gap), dt


@pytest.mark.parametrize("init,local,block", [(1, 4, 64), (0, 0, 64), (3, 2, 16), (2, 32, 64)])
def test_forced_page_mask_brute_force(init, local, block):
    """``forced_page_mask`` (pages.py:222-240) against a per-element loop of its
    contract: page p is forced for a query at absolute position t when p is a
    sink page (p < init_blocks) or lies in the local window ending at the
    query's page (qp - local_blocks <= p <= qp, qp = t // block_size); pages
    after qp are never local.  Covers 1-D and batched 2-D positions."""
    g = torch.Generator().manual_seed(init * 100 + local)
    num_pages = 11
    pos2 = torch.randint(0, num_pages * block, (3, 17), generator=g)
    pos2[0, :4] = torch.tensor([0, block - 1, block, num_pages * block - 1])
    for pos in (pos2[0], pos2):
        got = oracle.forced_page_mask(pos, num_pages=num_pages, block_size=block,
                                      init_blocks=init, local_blocks=local)
        P = pos.view(1, -1) if pos.ndim == 1 else pos
        assert got.shape == (P.shape[0], P.shape[1], num_pages)
        for b in range(P.shape[0]):
            for i in range(P.shape[1]):
                qp = int(P[b, i]) // block
                for p in range(num_pages):
                    want = p < init or (qp - local <= p <= qp)
                    assert bool(got[b, i, p]) == want, (b, i, p, qp)
