"""Decode on the GPU against the oracle: the cache append with incremental
compressed keys, stage-1 decode page plans, block-sparse attention over the
cache (split-K), the ``infllmv2_attn_with_kvcache`` drop-in, and the model's
decode step against a prefill of the same tokens where every page is kept.

Stage-1 plans are compared with the gap-aware checker at a one-step band (the
reference's stage-1 kernel is not vendored, so its summation order, and with
it the last bit of a bf16 score, is not pinned) and, as measured, must equal
the oracle's on every row."""
import pytest
import torch

import oracle
from leanselect_amd import minicpm
from leanselect_amd.infllm_v2 import (infllmv2_attn_stage1, infllmv2_attn_with_kvcache,
                                      max_pooling_1d_varlen)
from leanselect_amd.ops import compress_k, decode_topk_idx, kvcache_append, sparse_attention_kvcache
from leanselect_amd.ops.decode import n_windows

pytestmark = pytest.mark.gpu
DEV = "cuda"
G, D = 2, 128


def _cu(lens):
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return cu


def _i32(x):
    return torch.tensor(x, dtype=torch.int32, device=DEV)


def _filled_cache(lens, cap, seed=0, dtype=torch.bfloat16):
    """A cache holding ``lens`` random tokens per sequence, filled by one append
    from empty; returns (k, v, kc, packed K, packed V)."""
    B = len(lens)
    g = torch.Generator().manual_seed(seed)
    cu = _cu(lens)
    kp = torch.randn(cu[-1], G, D, generator=g).to(dtype)
    vp = torch.randn(cu[-1], G, D, generator=g).to(dtype)
    k = torch.zeros(B, cap, G, D, dtype=dtype, device=DEV)
    v = torch.zeros_like(k)
    kc = torch.zeros(B, n_windows(cap), G, D, dtype=dtype, device=DEV)
    kvcache_append(k, v, _i32([0] * B), kp.to(DEV), vp.to(DEV), _i32(cu), kc_cache=kc)
    return k, v, kc, kp, vp


def _gpu_windows(k_seq: torch.Tensor) -> torch.Tensor:
    """The prefill kernel's compressed keys of one sequence ``[L, G, D]``."""
    L = k_seq.shape[0]
    kc, _ = compress_k(k_seq.contiguous(), _i32([0, L]))
    return kc.cpu()


def test_append_fills_rows_and_windows_then_extends_them_token_by_token():
    lens = [37, 300, 1025, 0]
    cap = 1280
    k, v, kc, kp, vp = _filled_cache(lens, cap, seed=1)
    cu = _cu(lens)
    for b, L in enumerate(lens):
        assert torch.equal(k[b, :L].cpu(), kp[cu[b]:cu[b + 1]])
        assert torch.equal(v[b, :L].cpu(), vp[cu[b]:cu[b + 1]])
        n = n_windows(L)
        if n:
            assert torch.equal(kc[b, :n].cpu(), _gpu_windows(k[b, :L]))
            want = oracle.compress_k(kp[cu[b]:cu[b + 1]], [0, L])[0]
            assert (kc[b, :n].cpu() != want).float().mean().item() < 1e-3
    # Ragged decode steps (some sequences idle in some steps).
    g = torch.Generator().manual_seed(2)
    cur = list(lens)
    for step in range(70):
        n_new = [1, step % 3 == 0, 1, 1 if step < 40 else 0]
        n_new = [int(x) for x in n_new]
        tot = sum(n_new)
        kn = torch.randn(tot, G, D, generator=g).to(torch.bfloat16).to(DEV)
        vn = torch.randn(tot, G, D, generator=g).to(torch.bfloat16).to(DEV)
        kvcache_append(k, v, _i32(cur), kn, vn, _i32(_cu(n_new)), kc_cache=kc,
                       cache_seqlens_host=cur, cu_seqlens_new_host=_cu(n_new))
        cur = [c + n for c, n in zip(cur, n_new)]
    for b, L in enumerate(cur):
        n = n_windows(L)
        if n:  # windows formed one token at a time equal the prefill's of the same keys
            assert torch.equal(kc[b, :n].cpu(), _gpu_windows(k[b, :L])), b


@pytest.mark.parametrize("dtype,len_q", [(torch.bfloat16, 1), (torch.float16, 1),
                                         (torch.bfloat16, 3)])
def test_decode_select_matches_oracle(dtype, len_q):
    lens = [700, 3000, 9000, 64, 33, 129, 2049, 5000, 8191, 1000, 4500, 6666]
    cap = 9088
    k, v, kc, kp, vp = _filled_cache(lens, cap, seed=3, dtype=dtype)
    B, H = len(lens), 32
    g = torch.Generator().manual_seed(4)
    cu_q = _cu([len_q] * B)
    q = torch.randn(cu_q[-1], H, D, generator=g).to(dtype)
    for topk, local in [(64, 4), (16, 1), (96, 16)]:
        ids = decode_topk_idx(q.to(DEV), kc, _i32(lens), _i32(cu_q), topk=topk,
                              local_blocks=local, init_blocks=1).cpu()
        kc_packed = torch.cat([kc[b, :n_windows(L)].cpu() for b, L in enumerate(lens)])
        cu_kc = _cu([n_windows(L) for L in lens])
        want, pooled = oracle.decode_select(q, kc_packed, cu_q, cu_kc, lens,
                                            topk=topk, local_blocks=local, init_blocks=1,
                                            return_scores=True)
        assert ids.shape == want.shape
        rep = oracle.check_topk(ids, want, pooled, torch.bfloat16, ulp_band=1.0)
        print(f"decode select {dtype} len_q={len_q} topk={topk}: {rep}")
        assert rep.ok, str(rep)
        assert rep.exact_rows == rep.rows, str(rep)  # as measured: no row differs
        for gg in range(G):  # ascending kept ids, then -1 padding
            for b in range(cu_q[-1]):
                row = ids[gg, b].tolist()
                kept = [x for x in row if x >= 0]
                assert kept == sorted(set(kept)) and row == kept + [-1] * (len(row) - len(kept))


@pytest.mark.parametrize("lens,len_q", [
    ([131072, 50000, 7000, 300], 1),    # 2048 pages: one wave per row, gathered candidates
    ([70000, 20000], 3),                # 1141 pages, several rows per sequence
    ([600000, 20000], 1),               # 9375 pages: one workgroup per row, keys in LDS
])
def test_decode_select_long_rows_match_oracle(lens, len_q):
    cap = max(lens)
    k, v, kc, kp, vp = _filled_cache(lens, cap, seed=5)
    del k, v, kp, vp
    B, H = len(lens), 32
    g = torch.Generator().manual_seed(6)
    cu_q = _cu([len_q] * B)
    q = torch.randn(cu_q[-1], H, D, generator=g).to(torch.bfloat16)
    for topk, local in [(64, 4), (128, 1)]:
        ids = decode_topk_idx(q.to(DEV), kc, _i32(lens), _i32(cu_q), topk=topk,
                              local_blocks=local, init_blocks=1).cpu()
        kc_packed = torch.cat([kc[b, :n_windows(L)].cpu() for b, L in enumerate(lens)])
        cu_kc = _cu([n_windows(L) for L in lens])
        want, pooled = oracle.decode_select(q, kc_packed, cu_q, cu_kc, lens,
                                            topk=topk, local_blocks=local, init_blocks=1,
                                            return_scores=True)
        assert ids.shape == want.shape
        rep = oracle.check_topk(ids, want, pooled, torch.bfloat16, ulp_band=1.0)
        print(f"decode select lens={lens} len_q={len_q} topk={topk}: {rep}")
        assert rep.ok, str(rep)
        assert rep.exact_rows == rep.rows, str(rep)
        for gg in range(G):
            for r in range(cu_q[-1]):
                row = ids[gg, r].tolist()
                kept = [x for x in row if x >= 0]
                assert kept == sorted(set(kept)) and row == kept + [-1] * (len(row) - len(kept))


@pytest.mark.parametrize("lens", [[40000, 3000], [131072, 9000]])
def test_decode_select_all_scores_tied(lens):
    """Zero queries give every visible page the same stage-1 score: the top-k is
    decided by the tie rule alone (lower pages first, after the forced ones), and
    every key clears the lanes' bound, so the four-wave kernel hands the row to
    the one-wave selection."""
    cap = max(lens)
    k, v, kc, kp, vp = _filled_cache(lens, cap, seed=7)
    del k, v, kp, vp
    B, H = len(lens), 32
    cu_q = _cu([1] * B)
    q = torch.zeros(B, H, D, dtype=torch.bfloat16)
    ids = decode_topk_idx(q.to(DEV), kc, _i32(lens), _i32(cu_q), topk=64, local_blocks=4,
                          init_blocks=1).cpu()
    kc_packed = torch.cat([kc[b, :n_windows(L)].cpu() for b, L in enumerate(lens)])
    cu_kc = _cu([n_windows(L) for L in lens])
    want, pooled = oracle.decode_select(q, kc_packed, cu_q, cu_kc, lens, topk=64, local_blocks=4,
                                        init_blocks=1, return_scores=True)
    assert torch.equal(ids, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stage1_dropin_scores_match_oracle(dtype):
    """``infllmv2_attn_stage1(..., causal=False)`` on packed compressed keys
    against the oracle's stage-1 scores (rounded to the query dtype, 0 past a
    sequence's keys), including a NaN query row (0 everywhere, as the
    reference's wrapper maps NaN to 0) and a sequence without keys."""
    lens = [5000, 700, 20, 2100]  # 20 tokens: no compressed window
    B, H = len(lens), 32
    g = torch.Generator().manual_seed(31)
    nkc = [n_windows(L) for L in lens]
    cu_kc = _cu(nkc)
    kc = torch.randn(cu_kc[-1], G, D, generator=g).to(dtype)
    cu_q = _cu([2, 1, 1, 3])
    q = torch.randn(cu_q[-1], H, D, generator=g).to(dtype)
    q[4, 7, 3] = float("nan")
    max_k = max(nkc) + 5  # wider than every sequence: the tail is 0
    got = infllmv2_attn_stage1(q.to(DEV), kc.to(DEV), kc.to(DEV), cu_seqlens_q=_i32(cu_q),
                               cu_seqlens_k=_i32(cu_kc), cu_seqlens_v=_i32(cu_kc),
                               max_seqlen_q=3, max_seqlen_k=max_k, causal=False)
    assert got.shape == (G, cu_q[-1], max_k) and got.dtype == dtype
    raw = oracle.stage1_decode_scores(q, kc, cu_q, cu_kc)
    want = torch.zeros(G, cu_q[-1], max_k, dtype=torch.float64)
    want[..., : raw.shape[-1]] = raw
    want = torch.where(torch.isnan(want), torch.zeros_like(want), want).to(torch.float32).to(dtype)
    gf, wf = got.cpu().float(), want.float()
    # Softmax probabilities summed over 16 heads lie in [0, 16]: one rounding
    # step of the dtype at the value bounds the difference.
    tol = torch.tensor([oracle.dtype_step(float(x), dtype) for x in wf.flatten()]).view_as(wf)
    diff = (gf - wf).abs()
    print(f"\nstage1 drop-in {dtype}: max diff {diff.max().item():.3e}, "
          f"exact {(diff == 0).float().mean().item():.4f}")
    assert bool((diff <= tol + 1e-7).all())
    assert bool((got[0, 4].cpu() == 0).all())  # the NaN row (group 0 holds head 7)
    assert not bool(got.isnan().any())
    seq_of = [b for b in range(B) for _ in range(cu_q[b + 1] - cu_q[b])]
    for t, b in enumerate(seq_of):  # past the sequence's keys: exactly 0
        assert bool((got[:, t, nkc[b]:].cpu() == 0).all())
    with pytest.raises(NotImplementedError):
        infllmv2_attn_stage1(q.to(DEV), kc.to(DEV), kc.to(DEV), cu_seqlens_q=_i32(cu_q),
                             cu_seqlens_k=_i32(cu_kc), cu_seqlens_v=_i32(cu_kc),
                             max_seqlen_q=3, max_seqlen_k=max_k, causal=True)


def test_reference_decode_selection_from_the_dropins():
    """The reference's decode selection (compressed_attention with cache_lens,
    leanselect/models/minicpm.py:617-705) composed from the drop-ins alone --
    stage-1 scores, bf16, max_pooling_1d_varlen, top-k, sort, ids past the
    row's page to -1 -- gives ``decode_topk_idx``'s plans (gap-aware: the
    composition's torch.topk breaks ties its own way)."""
    lens = [40000, 9000, 3000]
    cap = max(lens)
    k, v, kc_cache, _, _ = _filled_cache(lens, cap, seed=33)
    del k, v
    B, H, bs, topk, local, init = len(lens), 32, 64, 64, 4, 1
    g = torch.Generator().manual_seed(34)
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(DEV)
    cu_q = list(range(B + 1))
    nkc = [n_windows(L) for L in lens]
    cu_kc = _cu(nkc)
    kc = torch.cat([kc_cache[b, :nkc[b]] for b in range(B)])
    cache_lens = [L - 1 for L in lens]  # the reference's cache_lens = seq_lens_k - 1
    score = infllmv2_attn_stage1(q, kc, kc, cu_seqlens_q=_i32(cu_q), cu_seqlens_k=_i32(cu_kc),
                                 cu_seqlens_v=_i32(cu_kc), max_seqlen_q=1,
                                 max_seqlen_k=max(nkc), causal=False)
    score = score.to(torch.bfloat16)
    block = max_pooling_1d_varlen(score.contiguous(), _i32(cu_q), _i32(cu_kc), _i32(cache_lens),
                                  1, max(nkc), local_blocks=local, init_blocks=init,
                                  block_size=bs, stride=16)
    kk = min(topk, block.shape[-1])
    comp = block.topk(kk, dim=-1).indices.sort(-1).values
    q_idx = torch.tensor([c // bs for c in cache_lens], device=DEV)
    comp[comp > q_idx[None, :, None]] = -1
    comp = comp.to(torch.int32)
    ids = decode_topk_idx(q, kc_cache, _i32(lens), _i32(cu_q), topk=topk, local_blocks=local,
                          init_blocks=init)
    assert comp.shape == ids.shape
    rep = oracle.check_topk(comp.cpu(), ids.cpu(), block.cpu().double(), torch.bfloat16,
                            ulp_band=1.0)
    print(f"\nreference decode selection from the drop-ins: {rep}")
    assert rep.ok, str(rep)


def _packed(k, v, lens):
    return (torch.cat([k[b, :L].cpu() for b, L in enumerate(lens)]),
            torch.cat([v[b, :L].cpu() for b, L in enumerate(lens)]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_attention_matches_oracle(dtype):
    lens = [700, 3000, 9000, 65]
    cap = 9088
    k, v, kc, _, _ = _filled_cache(lens, cap, seed=5, dtype=dtype)
    B, H = len(lens), 32
    g = torch.Generator().manual_seed(6)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    cu_q = list(range(B + 1))
    ids = decode_topk_idx(q.to(DEV), kc, _i32(lens), _i32(cu_q), topk=64, local_blocks=4)
    kpk, vpk = _packed(k, v, lens)
    want = oracle.sparse_attention(q, kpk, vpk, cu_q, _cu(lens), ids.cpu(), causal=False)[0]
    for n_splits in (None, 1, 7, ids.shape[2]):
        out = sparse_attention_kvcache(q.to(DEV), k, v, _i32(lens), ids, _i32(cu_q),
                                       n_splits=n_splits)
        ok, mx, mr = oracle.check_attention(out.cpu(), want)
        print(f"decode attention {dtype} splits={n_splits}: max {mx:.3e} mean rel {mr:.3e}")
        assert ok, (n_splits, mx, mr)
    # A messy plan: -1, repeats, ids past the sequence, unsorted.
    T = 20
    messy = torch.randint(-2, 160, (G, B, T), generator=g, dtype=torch.int32)
    messy[:, :, 5] = messy[:, :, 2]
    out, lse = sparse_attention_kvcache(q.to(DEV), k, v, _i32(lens), messy.to(DEV), _i32(cu_q),
                                        return_lse=True)
    want, want_lse = oracle.sparse_attention(q, kpk, vpk, cu_q, _cu(lens), messy, causal=False)
    ok, mx, mr = oracle.check_attention(out.cpu(), want)
    assert ok, (mx, mr)
    fin = torch.isfinite(want_lse)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert torch.allclose(lse.cpu()[fin].double(), want_lse[fin].double(), rtol=0, atol=1e-4)


def test_decode_attention_several_rows_per_sequence_causal():
    # Rows of a multi-token step: row i of sequence b sees keys j <= len_b - len_q(b) + i.
    lens = [300, 1100]
    cap = 1152
    k, v, kc, _, _ = _filled_cache(lens, cap, seed=7)
    lq = [3, 5]
    cu_q = _cu(lq)
    g = torch.Generator().manual_seed(8)
    q = torch.randn(cu_q[-1], 32, D, generator=g).to(torch.bfloat16)
    ids = decode_topk_idx(q.to(DEV), kc, _i32(lens), _i32(cu_q), topk=8, local_blocks=1)
    kpk, vpk = _packed(k, v, lens)
    for causal in (True, False):
        out = sparse_attention_kvcache(q.to(DEV), k, v, _i32(lens), ids, _i32(cu_q), causal=causal)
        want = oracle.sparse_attention(q, kpk, vpk, cu_q, _cu(lens), ids.cpu(), causal=causal)[0]
        ok, mx, mr = oracle.check_attention(out.cpu(), want)
        assert ok, (causal, mx, mr)


def test_with_kvcache_dropin_appends_and_attends():
    B, cap, H = 2, 512, 32
    lens = [100, 333]
    k, v, kc, _, _ = _filled_cache(lens, cap, seed=9)
    g = torch.Generator().manual_seed(10)
    q = torch.randn(B, 1, H, D, generator=g).to(torch.bfloat16).to(DEV)
    kn = torch.randn(B, 1, G, D, generator=g).to(torch.bfloat16).to(DEV)
    vn = torch.randn(B, 1, G, D, generator=g).to(torch.bfloat16).to(DEV)
    pages = torch.tensor([[0, 1], [0, 5]], dtype=torch.int32)  # per sequence
    ids = pages[None].expand(G, B, 2).contiguous().to(DEV)
    out, lse = infllmv2_attn_with_kvcache(q, k, v, kn, vn, cache_seqlens=_i32(lens),
                                          topk_idx=ids, return_softmax_lse=True)
    assert out.shape == (B, 1, H, D) and lse.shape == (B, H, 1)
    new_lens = [L + 1 for L in lens]
    for b in range(B):
        assert torch.equal(k[b, lens[b]], kn[b, 0]) and torch.equal(v[b, lens[b]], vn[b, 0])
    kpk, vpk = _packed(k, v, new_lens)
    want = oracle.sparse_attention(q.view(B, H, D).cpu(), kpk, vpk, list(range(B + 1)),
                                   _cu(new_lens), ids.cpu(), causal=False)[0]
    ok, mx, mr = oracle.check_attention(out.view(B, H, D).cpu(), want)
    assert ok, (mx, mr)
    # No plan: every page.
    dense = infllmv2_attn_with_kvcache(q, k, v, cache_seqlens=_i32(new_lens))
    all_ids = torch.arange(6, dtype=torch.int32).expand(G, B, 6).contiguous()
    want = oracle.sparse_attention(q.view(B, H, D).cpu(), kpk, vpk, list(range(B + 1)),
                                   _cu(new_lens), all_ids, causal=False)[0]
    ok, mx, mr = oracle.check_attention(dense.view(B, H, D).cpu(), want)
    assert ok, (mx, mr)


def test_with_kvcache_dense_beyond_256_pages():
    """``topk_idx=None`` over caches of more than 256 pages (16384 tokens): the
    pages are attended in groups merged by their log-sum-exp, against the oracle
    over every page; a short sequence beside a long one has groups with no key."""
    B, cap, H = 2, 20480, 16
    lens = [20000, 5000]
    k, v, _, kp, vp = _filled_cache(lens, cap, seed=21)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(B, 1, H, D, generator=g).to(torch.bfloat16).to(DEV)
    out, lse = infllmv2_attn_with_kvcache(q, k, v, cache_seqlens=_i32(lens),
                                          return_softmax_lse=True)
    n_pages = -(-max(lens) // 64)
    all_ids = torch.arange(n_pages, dtype=torch.int32).expand(G, B, n_pages).contiguous()
    want, want_lse = oracle.sparse_attention(q.view(B, H, D).cpu(), kp, vp, list(range(B + 1)),
                                             _cu(lens), all_ids, causal=False)
    ok, mx, mr = oracle.check_attention(out.view(B, H, D).cpu(), want)
    print(f"\ndense kvcache {lens}: max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert ok, (mx, mr)
    got_lse = lse.permute(1, 0, 2).reshape(H, B).cpu().double()
    torch.testing.assert_close(got_lse, want_lse.double(), rtol=0, atol=2e-3)


def test_model_decode_matches_prefill_when_every_page_is_kept():
    # With a budget above the page count both selectors keep every page, so a
    # decode step must give the logits of a prefill of the extended sequences.
    cfg = minicpm.MiniCPMConfig(hidden_size=1024, num_hidden_layers=2, num_attention_heads=8,
                                num_key_value_heads=2, intermediate_size=2048, vocab_size=4096,
                                topk=64, local_blocks=4)
    model = minicpm.MiniCPMLeanSelect(cfg, device=DEV, seed=3)
    lens = [300, 517]
    g = torch.Generator(device=DEV).manual_seed(11)
    steps = 6
    toks = [torch.randint(0, cfg.vocab_size, (L + steps,), generator=g, device=DEV,
                          dtype=torch.int32) for L in lens]
    cache = model.new_cache(len(lens), 1024)
    cu = _cu(lens)
    model.prefill(torch.cat([t[:L] for t, L in zip(toks, lens)]), cu, cache=cache)
    assert cache.lengths == lens
    worst = 0.0
    for s in range(steps):
        ids = torch.stack([t[L + s] for t, L in zip(toks, lens)])
        got = model.decode_step(ids, cache)
        cur = [L + s + 1 for L in lens]
        want = model.prefill(torch.cat([t[:n] for t, n in zip(toks, cur)]), _cu(cur))
        rel = ((got - want).abs().max() / want.abs().max()).item()
        worst = max(worst, rel)
        assert torch.isfinite(got).all()
        assert rel < 3e-2, (s, rel)
    print(f"decode vs prefill logits: worst max-rel {worst:.3e}")
    assert cache.lengths == [L + steps for L in lens]
