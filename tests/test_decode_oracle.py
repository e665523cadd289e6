"""Decode oracle pins and decode host-side checks (CPU only).

The incremental compressed-key update is pinned by equality with the prefill
compression of the same keys; the stage-1 decode scores by the invariants that
fix softmax-summed-over-the-group (rows sum to the group size, one key gives it
exactly) and by ``torch.softmax`` as the library routine; the decode plan tail
by brute force over small rows.  The kernel's own division by the group size,
if any, is not visible in the reference (a power of two: rankings do not
depend on it) and its summation order is unpinned.
"""
import math
import random

import pytest
import torch

import oracle
from leanselect_amd.ops import decode as dec


@pytest.mark.parametrize("first,steps", [(0, [1] * 70), (10, [1] * 60), (31, [1] * 40),
                                         (32, [1] * 40), (33, [3, 1, 7, 16, 1, 1, 30]),
                                         (100, [1] * 50), (257, [64, 1, 1, 2])])
def test_incremental_windows_equal_prefill_compression(first, steps):
    g = torch.Generator().manual_seed(first)
    total = first + sum(steps)
    k = torch.randn(total, 2, 16, generator=g).to(torch.bfloat16)
    inc = oracle.cache_windows_incremental(k, [first] + steps)
    full, cu = oracle.compress_k(k, [0, total])
    assert inc.shape == full.shape == (oracle.n_windows(total), 2, 16)
    assert torch.equal(inc, full)


def test_window_count_matches_closed_form():
    for L in range(0, 200):
        assert oracle.n_windows(L) == (0 if L < 32 else (L - 32) // 16 + 1)
        assert dec.n_windows(L) == oracle.n_windows(L)


def _toy(seed, lens, H=8, G=2, D=32, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    ncs = [oracle.n_windows(L) for L in lens]
    cu_kc = [0]
    for n in ncs:
        cu_kc.append(cu_kc[-1] + n)
    kc = torch.randn(cu_kc[-1], G, D, generator=g).to(dtype)
    q = torch.randn(len(lens), H, D, generator=g).to(dtype)
    return q, kc, cu_kc


def test_stage1_rows_sum_to_group_size_and_match_torch_softmax():
    lens = [40, 300, 1000]
    q, kc, cu_kc = _toy(0, lens)
    cu_q = list(range(len(lens) + 1))
    s = oracle.stage1_decode_scores(q, kc, cu_q, cu_kc)
    G, H, D = kc.shape[1], q.shape[1], q.shape[2]
    gs = H // G
    for b in range(len(lens)):
        n = cu_kc[b + 1] - cu_kc[b]
        assert torch.allclose(s[:, b, :n].sum(-1), torch.full((G,), float(gs), dtype=torch.float64))
        assert bool((s[:, b, n:] == 0).all())
        for g in range(G):
            logits = (q[b, g * gs:(g + 1) * gs].float() @ kc[cu_kc[b]:cu_kc[b + 1], g].float().T) * D ** -0.5
            ref = torch.softmax(logits, dim=-1).sum(0)
            assert torch.allclose(s[g, b, :n].float(), ref, rtol=1e-5, atol=1e-6)


def test_stage1_single_key_gives_group_size():
    q, kc, cu_kc = _toy(1, [32, 32])
    s = oracle.stage1_decode_scores(q, kc, [0, 1, 2], cu_kc)
    assert s.shape == (2, 2, 1)
    assert bool((s == 4.0).all())


def _brute_plan(pooled_row, take, q_idx):
    order = sorted(range(len(pooled_row)), key=lambda p: (-pooled_row[p], p))[:take]
    kept = sorted(p for p in order if p <= q_idx)
    return kept + [-1] * (take - len(kept))


def test_decode_select_tail_by_brute_force():
    lens = [50, 200, 700, 1300]
    q, kc, cu_kc = _toy(2, lens)
    cu_q = list(range(len(lens) + 1))
    for topk, local in [(4, 1), (8, 2), (64, 2)]:
        ids, pooled = oracle.decode_select(q, kc, cu_q, cu_kc, lens, topk=topk, local_blocks=local,
                                           init_blocks=1, return_scores=True)
        out_len = pooled.shape[-1]
        assert out_len == math.ceil(max(lens) / 64)
        take = min(topk, out_len)
        assert ids.shape == (kc.shape[1], len(lens), take)
        for g in range(ids.shape[0]):
            for b, L in enumerate(lens):
                q_idx = (L - 1) // 64
                row = pooled[g, b].tolist()
                assert ids[g, b].tolist() == _brute_plan(row, take, q_idx)
                # sink and local pages are forced (+inf) and kept whenever they fit
                forced = [p for p in range(out_len) if row[p] == math.inf]
                assert forced == sorted({0} | set(range(max(0, q_idx - local), q_idx + 1)))


def test_decode_select_pooling_reads_only_the_rows_own_windows():
    # A shorter sequence's pooled pages past its windows are -inf even though the
    # score rows are padded to the longest sequence's width.
    lens = [100, 900]
    q, kc, cu_kc = _toy(3, lens)
    ids, pooled = oracle.decode_select(q, kc, [0, 1, 2], cu_kc, lens, topk=16, local_blocks=0,
                                       init_blocks=0, return_scores=True)
    q_idx0 = (lens[0] - 1) // 64
    assert bool((pooled[:, 0, q_idx0 + 1:] == -math.inf).all())
    assert all(int(p) <= q_idx0 for p in ids[:, 0].flatten() if p >= 0)


# ---- host-side argument checks (raise before any GPU call) -----------------
def _cache(B=2, cap=128, G=2, D=128, dtype=torch.bfloat16):
    return torch.zeros(B, cap, G, D, dtype=dtype), torch.zeros(B, cap, G, D, dtype=dtype)


def test_append_rejects_capacity_overflow_and_bad_offsets():
    k, v = _cache()
    lens = torch.tensor([120, 0], dtype=torch.int32)
    new = torch.zeros(10, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="capacity"):
        dec.kvcache_append(k, v, lens, new, new, torch.tensor([0, 10, 10], dtype=torch.int32))
    with pytest.raises(ValueError, match="offsets"):
        dec.kvcache_append(k, v, lens, new, new, torch.tensor([0, 4, 9], dtype=torch.int32))
    with pytest.raises(ValueError, match="int32"):
        dec.kvcache_append(k, v, lens.long(), new, new, torch.tensor([0, 0, 10], dtype=torch.int32))
    with pytest.raises(ValueError, match="bf16 or fp16"):
        dec.kvcache_append(k.float(), v.float(), lens, new.float(), new.float(),
                           torch.tensor([0, 0, 10], dtype=torch.int32))


def test_append_rejects_a_too_small_compressed_cache():
    k, v = _cache(B=1, cap=256)
    kc = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)  # 4 windows < 14 needed for 240 tokens
    new = torch.zeros(240, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="kc_capacity"):
        dec.kvcache_append(k, v, torch.tensor([0], dtype=torch.int32), new, new,
                           torch.tensor([0, 240], dtype=torch.int32), kc_cache=kc)


def test_decode_select_and_attention_reject_bad_shapes():
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    kc = torch.zeros(2, 10, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="hold its query rows"):
        dec.decode_topk_idx(q, kc, torch.tensor([0, 5], dtype=torch.int32),
                            torch.tensor([0, 1, 2], dtype=torch.int32), topk=8)
    with pytest.raises(ValueError, match="fewer windows"):
        dec.decode_topk_idx(q, kc, torch.tensor([1000, 5], dtype=torch.int32),
                            torch.tensor([0, 1, 2], dtype=torch.int32), topk=8)
    k, v = _cache()
    with pytest.raises(ValueError, match="topk_idx"):
        dec.sparse_attention_kvcache(q, k, v, torch.tensor([5, 5], dtype=torch.int32),
                                     torch.zeros(2, 3, 4, dtype=torch.int32),
                                     torch.tensor([0, 1, 2], dtype=torch.int32))
    with pytest.raises(ValueError, match="int32"):
        dec.sparse_attention_kvcache(q, k, v, torch.tensor([5, 5]),
                                     torch.zeros(2, 2, 4, dtype=torch.int32),
                                     torch.tensor([0, 1, 2], dtype=torch.int32))


def test_decode_out_len_matches_the_pooling_width():
    assert dec.decode_out_len([1, 64, 65], [1, 1, 1]) == 2
    assert dec.decode_out_len([128, 300], [1, 4]) == 5  # ceil((4 + max(127, 296)) / 64)
    random.seed(0)
    for _ in range(50):
        lens = [random.randint(1, 5000) for _ in range(3)]
        lq = [random.randint(1, min(8, L)) for L in lens]
        want = (max(lq) + max(L - q for L, q in zip(lens, lq)) + 63) // 64
        assert dec.decode_out_len(lens, lq) == want
