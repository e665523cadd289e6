"""Pins the NOSA oracle (CPU): CIS pooling against the reference's own
``avg_pool1d`` check, page pooling against LeanSelect's 5-atom page max and a
brute-force loop, the two-stage selection against a loop restatement, and the
one-pass attention against the reference's numerator / denominator form."""
import math

import pytest
import torch

import oracle


def _cu(lens):
    return torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0).tolist()), dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mean_pooling_matches_avg_pool1d(dtype):
    # The reference's self-test (cis_pooling.py:75-103): lens 67 and 1432, H 4,
    # against avg_pool1d per sequence, broadcast to the sequence's rows.
    torch.manual_seed(0)
    lens = [67, 1432]
    cu = _cu(lens)
    N, H = sum(lens), 4
    cis = torch.randn(N, H).to(dtype)
    got = oracle.nosa_mean_pooling(cis, cu, max(lens))
    M = max(lens) // 16 - 1
    assert got.shape == (H, N, M)
    want = torch.zeros(H, N, M, dtype=torch.float64)
    for b in range(2):
        s, e = int(cu[b]), int(cu[b + 1])
        pooled = torch.nn.functional.avg_pool1d(cis[s:e].T.unsqueeze(0).double(), 32, 16)[0]
        want[:, s:e, : pooled.shape[-1]] = pooled[:, None, :]
    assert torch.equal(got, want.to(dtype))


def _pool_loop(row, lk, out_len, off_bq, init, local):
    out = []
    for p in range(out_len):
        if p < init or (off_bq - local <= p <= off_bq):
            out.append(math.inf)
            continue
        vals = [row[j] for j in range(4 * p - 1, 4 * p + 4) if 0 <= j < lk]
        out.append(max(vals) if vals else -math.inf)
    return out


def test_page_pooling_brute_force_and_leanselect_window():
    torch.manual_seed(1)
    lens_q, lens_k = [70, 300, 5], [3, 17, 0]  # compressed key counts
    cq, ck = _cu(lens_q), _cu(lens_k)
    Hk, T, max_k = 2, sum(lens_q), max(lens_k)
    inp = torch.randn(Hk, T, max_k, dtype=torch.float64)
    cache = torch.tensor([0, 64, 3])
    got = oracle.page_maxpool_varlen(inp, cq, ck, cache, max(lens_q), max_k, local_blocks=2,
                                     init_blocks=1)
    out_len = (max(lens_q) + 64 + 63) // 64
    assert got.shape == (Hk, T, out_len)
    for b in range(3):
        for t in range(int(cq[b]), int(cq[b + 1])):
            off_bq = (t - int(cq[b]) + int(cache[b])) // 64
            for h in range(Hk):
                want = _pool_loop(inp[h, t].tolist(), lens_k[b], out_len, off_bq, 1, 2)
                assert got[h, t].tolist() == want
    # Non-forced pages pool exactly like LeanSelect's page max (pages.py:146-187).
    row = inp[0, 100]
    ls = oracle.pool_atoms_to_pages(row[: lens_k[1]], seq_len=64 * out_len)
    p = oracle.page_maxpool_varlen(inp[:, 100:101], torch.tensor([0, 1]), torch.tensor([0, lens_k[1]]),
                                   torch.tensor([0]), 64 * out_len, max_k, local_blocks=0, init_blocks=0)
    free = [j for j in range(out_len) if j != 0]  # page 0 is the row's own (forced) page
    assert torch.equal(p[0, 0, free], ls[free])


def _select_loop(block_row, cis_row, q_idx, topk, n_short):
    out_len = len(block_row)
    order_qk = sorted(range(out_len), key=lambda p: (-block_row[p], p))
    short = set(order_qk[: min(n_short, out_len)])
    cis = [(-math.inf if p > q_idx else cis_row[p]) for p in range(out_len)]
    cis = [math.inf if p in short else c for p, c in enumerate(cis)]
    order = sorted(range(out_len), key=lambda p: (-cis[p], p))[: min(topk, out_len)]
    ids = sorted(order)
    return [(-1 if p > q_idx else p) for p in ids]


@pytest.mark.parametrize("clip", ["sequence", "row"])
def test_nosa_selection_loop_restatement(clip):
    torch.manual_seed(2)
    lens = [2000, 700]  # the short sequence has 11 pages of real windows
    cq = _cu(lens)
    ck = _cu([(n - 32) // 16 + 1 for n in lens])
    G, max_kc = 2, int((ck[1:] - ck[:-1]).max())
    atom = torch.randn(G, sum(lens), max_kc).to(torch.bfloat16).double()
    for b in range(2):
        atom[:, int(cq[b]) : int(cq[b + 1]), int(ck[b + 1] - ck[b]):] = float("-inf")
    cis = torch.randn(sum(lens), G).to(torch.bfloat16)
    ids, block, over = oracle.nosa_select_prefill(
        atom, cis, cq, ck, cq, max(lens), max(lens), topk=12, init_blocks=1, local_blocks=2,
        select_blocks=3, return_scores=True, clip=clip)
    q_idx = oracle.nosa_q_idx(cq, max(lens))
    score_cis = oracle.nosa_mean_pooling(cis, cq, max(lens))
    out_len = (max(lens) + 63) // 64
    n_differ = 0
    for r in range(0, sum(lens), 7):
        b = 0 if r < lens[0] else 1
        lk = int(ck[b + 1] - ck[b])
        off = (r - int(cq[b])) // 64
        for g in range(G):
            # The row clip pools the padded row: max_kc atom columns (-inf padding)
            # and max(lens) // 16 - 1 window means (0 padding).
            lk_qk = max_kc if clip == "row" else lk
            lk_cis = score_cis.shape[-1] if clip == "row" else lk
            brow = _pool_loop(atom[g, r].tolist(), lk_qk, out_len, off, 1, 2)
            crow = _pool_loop(score_cis[g, r].double().tolist(), lk_cis, out_len, off, 1, 2)
            want = _select_loop(brow, crow, int(q_idx[r]), 12, 1 + 2 + 3)
            assert ids[g, r].tolist() == want, (r, g)
            if clip == "row":
                crow_seq = _pool_loop(score_cis[g, r].double().tolist(), lk, out_len, off, 1, 2)
                n_differ += want != _select_loop(brow, crow_seq, int(q_idx[r]), 12, 1 + 2 + 3)
    if clip == "row":  # the short sequence's late pages score 0 instead of -inf
        assert n_differ > 0


def test_nosa_attention_is_numerator_over_denominator():
    torch.manual_seed(3)
    lens = [300, 90]
    cq = _cu(lens)
    N, H, G, D = sum(lens), 4, 2, 16
    q, k, v = (torch.randn(N, n, D, dtype=torch.float64) for n in (H, G, G))
    cis = torch.randn(N, G, dtype=torch.float64)
    T = 3
    ids = torch.full((G, N, T), -1, dtype=torch.int32)
    for t in range(N):
        b = 0 if t < lens[0] else 1
        qp = (t - int(cq[b])) // 64
        pages = sorted({0, qp, max(qp - 2, 0)})
        ids[:, t, : len(pages)] = torch.tensor(pages, dtype=torch.int32)
    got = oracle.nosa_attention(q, k, v, cis, cq, cq, ids, block_size=64)
    w = torch.exp(cis)
    num, _ = oracle.sparse_attention(q, k, v * w[:, :, None], cq, cq, ids)
    den, _ = oracle.sparse_attention(q, k, w[:, :, None].expand(N, G, D).contiguous(), cq, cq, ids)
    torch.testing.assert_close(got, num / den[..., :1], rtol=1e-12, atol=1e-12)


def test_q_idx_is_aligned_to_the_longest_sequence():
    # nosa.py:1175-1189: rows of a shorter sequence are shifted to end with the
    # longest one (a property of the reference kept as is).
    q = oracle.nosa_q_idx(_cu([70, 131]), 131)
    assert q[:4].tolist() == [0, 0, 0, 1]          # (t + 61) // 64
    assert q[69].item() == (69 + 61) // 64 == 2
    assert q[70:72].tolist() == [0, 0] and q[-1].item() == 130 // 64


def test_page_maxpool_of_zero_width_scores_is_the_forced_overlay():
    """No score column at all (every sequence shorter than a CIS window): every page
    pools an empty range (-inf) and only the forced pages remain (+inf)."""
    cu = torch.tensor([0, 20, 23, 54])
    out = oracle.page_maxpool_varlen(torch.zeros(2, 54, 0), cu, cu, torch.zeros(3, dtype=torch.int32),
                                     31, 31, local_blocks=2, init_blocks=1)
    assert out.shape == (2, 54, 1)
    assert bool(torch.isposinf(out).all())  # page 0 is the sink page of every row
    out = oracle.page_maxpool_varlen(torch.zeros(1, 54, 0), cu, cu, torch.zeros(3, dtype=torch.int32),
                                     31, 31, local_blocks=0, init_blocks=0)
    assert bool(torch.isposinf(out).all())  # page 0 is each row's own local page


def test_page_pooling_clips_to_each_sequence_and_the_choice_is_visible():
    """The window of a row is clipped to its own sequence's score columns
    (``cu_seqlens_k``), not to the padded width ``max_seqlen_k``.  The
    reference's ``max_pooling_1d_varlen(input, cu_seqlens_q, cu_seqlens_k, ...,
    max_seqlen_k, ...)`` (paper1.patch:2664-2760) receives the padded width
    separately (it asserts ``input.shape[2] == max_seqlen_k``), so the per-sequence
    offsets serve only to bound each sequence's columns.  Padding columns are
    nonzero here, so the other clip gives a different answer and the check has
    teeth."""
    lens_q, lens_k = [300, 300], [9, 17]
    cq, ck = _cu(lens_q), _cu(lens_k)
    max_k = max(lens_k)
    inp = torch.full((1, 600, max_k), -5.0, dtype=torch.float64)
    inp[:, :300, 9:] = 7.0  # the first sequence's padding columns: larger than any score
    got = oracle.page_maxpool_varlen(inp, cq, ck, torch.zeros(2, dtype=torch.int32), 300, max_k,
                                     local_blocks=0, init_blocks=0)
    out_len = (300 + 63) // 64
    t = 299  # last row of sequence 0, page 4 (forced); pages 0..3 are pooled
    own = _pool_loop(inp[0, t].tolist(), lens_k[0], out_len, 4, 0, 0)
    padded = _pool_loop(inp[0, t].tolist(), max_k, out_len, 4, 0, 0)
    assert got[0, t].tolist() == own
    assert own != padded  # page 2 reads column 9 under the max_k clip
    assert own[2] == -5.0 and padded[2] == 7.0 and own[3] == -math.inf
    # clip="row" is the padded loop; for the longest sequence both clips agree.
    got_row = oracle.page_maxpool_varlen(inp, cq, ck, torch.zeros(2, dtype=torch.int32), 300,
                                         max_k, local_blocks=0, init_blocks=0, clip="row")
    assert got_row[0, t].tolist() == padded
    assert torch.equal(got_row[:, 300:], got[:, 300:])
    with pytest.raises(ValueError, match="clip"):
        oracle.page_maxpool_varlen(inp, cq, ck, torch.zeros(2, dtype=torch.int32), 300, max_k,
                                   local_blocks=0, init_blocks=0, clip="max_k")


def test_nosa_checker_flags_differences_without_a_tie():
    # One row, out_len 8, q_idx 7: shortlist of 3 qk pages, then the 4 best CIS pages.
    inf = math.inf
    block = torch.tensor([[[inf, 5.0, 4.0, 3.0, 2.0, 1.0, 0.5, inf]]], dtype=torch.float64)
    cis = torch.tensor([[[inf, 0.1, 0.2, 0.9, 0.8, 0.3, 0.7, inf]]], dtype=torch.float64)
    q_idx = torch.tensor([7])
    ids, b, over = oracle.nosa_two_stage(block, cis, q_idx, topk=4, qk_select=3,
                                         return_scores=True)
    assert ids.tolist() == [[[0, 1, 3, 7]]]  # shortlist {0, 7, 1}, then CIS 0.9 (page 3)
    rep = oracle.check_nosa_topk(ids, ids, b, over, topk=4, qk_select=3)
    assert rep.ok and rep.exact_rows == 1
    wrong = torch.tensor([[[0, 1, 4, 7]]], dtype=torch.int32)  # 0.8 < 0.9: no tie
    assert not oracle.check_nosa_topk(wrong, ids, b, over, topk=4, qk_select=3).ok
    # A tie at the stage-2 boundary admits the other page.
    cis_tie = cis.clone()
    cis_tie[0, 0, 4] = 0.9
    ids2, b2, over2 = oracle.nosa_two_stage(block, cis_tie, q_idx, topk=4, qk_select=3,
                                            return_scores=True)
    rep = oracle.check_nosa_topk(wrong, ids2, b2, over2, topk=4, qk_select=3)
    assert rep.ok and rep.band_rows == 1
    # A tie at the shortlist boundary (qk 4.0 vs 4.0) admits the other shortlist.
    blk_tie = block.clone()
    blk_tie[0, 0, 3] = 5.0
    ids3, b3, over3 = oracle.nosa_two_stage(blk_tie, cis, q_idx, topk=4, qk_select=3,
                                            return_scores=True)
    other = torch.tensor([[[0, 3, 4, 7]]], dtype=torch.int32)
    assert oracle.check_nosa_topk(other, ids3, b3, over3, topk=4, qk_select=3).ok
    # A row with a different id count always fails.
    short = torch.tensor([[[0, 1, 3, -1]]], dtype=torch.int32)
    assert not oracle.check_nosa_topk(short, ids2, b2, over2, topk=4, qk_select=3).ok


def test_window_means_are_the_broadcast_rows():
    torch.manual_seed(5)
    lens = [33, 100, 7, 400]
    cu = _cu(lens)
    cis = torch.randn(sum(lens), 2).to(torch.bfloat16)
    full = oracle.nosa_mean_pooling(cis, cu, max(lens))
    for b in range(len(lens)):
        s, e = int(cu[b]), int(cu[b + 1])
        row = oracle.nosa_window_means(cis, s, e, max(lens))
        for t in range(s, e):
            assert torch.equal(full[:, t], row)
