"""Pins the oracle's NaN / infinity rule of the prefill selection
(leanselect/models/minicpm.py:3124-3141: forced pages at +inf, ``torch.topk``
ranking NaN above +inf, chosen pages with a NaN or -inf score emitted as -1)
against the reference's own torch formulation (``oracle.reference_path``:
einsums, ``max_pool1d`` and ``torch.topk`` on the CPU), on a layer whose query
and key rows carry planted NaN and infinities.  Rows are compared as sets of
valid ids plus the number of -1 slots, which ``torch.topk``'s unspecified order
among equal (or NaN) values cannot change.  A planted mistake in the oracle
(NaN ranked below every number) must be caught."""
import math

import pytest
import torch

import oracle
from oracle import leanselect_oracle
from leanselect_amd import workloads


def _masters(sel):
    return [getattr(sel, n).detach().float()
            for n in ("head_mix", "kv_head_mix", "q_proj", "k_proj")]


def _planted_case():
    # Budget 8 = 1 sink + 3 local + 4 others, so a row with more than 4 NaN pages
    # loses its forced pages too.
    case = workloads.head_space_layer(1024, seed=9, topk=8, local_blocks=2)
    q, k = case.q.clone(), case.k.clone()
    nan, inf = float("nan"), float("inf")
    q[900, 5, 3] = nan        # every score of row 900's group 1 (heads 4..7) is NaN
    q[800, 0, 7] = nan        # group 0 of row 800
    q[850, 5, 1] = inf        # +inf and -inf (and NaN where they cancel) for group 1
    q[950, 1, 9] = -inf
    k[64 * 3 + 5, 0, 11] = nan  # the windows over key 197: NaN for every later row, group 0
    k[64 * 9 + 40, 1, 2] = inf
    return case, q, k


def _rows_as_sets(ids, rows):
    out = {}
    for g in range(ids.shape[0]):
        for r in rows:
            row = ids[g, r].tolist()
            out[g, r] = (sorted(x for x in row if x >= 0), sum(1 for x in row if x < 0))
    return out


def _plans(case, q, k):
    kc, cu_c = oracle.compress_k(k, case.cu_host)
    qf, kf = oracle.fused_weights(*_masters(case.selector), torch.float32)
    want, scores = oracle.select_prefill(q, kc, case.cu_host, cu_c.tolist(), qf, kf,
                                         topk=case.topk, init_blocks=case.init_blocks,
                                         local_blocks=case.local_blocks, return_scores=True)
    ref = oracle.reference_select_prefill(q, kc, case.cu_host, cu_c.tolist(),
                                          _masters(case.selector), topk=case.topk,
                                          init_blocks=case.init_blocks,
                                          local_blocks=case.local_blocks)
    return want, ref, scores


def test_nan_and_inf_rows_match_the_reference_torch_path():
    case, q, k = _planted_case()
    want, ref, scores = _plans(case, q, k)
    # Rows whose visible, non-forced page scores hold a NaN or an infinity.
    special = sorted({int(r) for g in range(scores.shape[0])
                      for r in torch.nonzero(torch.isnan(scores[g]).any(-1)
                                             | torch.isinf(scores[g]).sum(-1).gt(
                                                 scores.shape[-1])).flatten().tolist()}
                     | {800, 850, 900, 950} | set(range(64 * 3, 1024, 97)))
    got_w, got_r = _rows_as_sets(want, special), _rows_as_sets(ref, special)
    bad = []
    for key in got_w:
        (ids_w, n_w), (ids_r, n_r) = got_w[key], got_r[key]
        if n_w != n_r:
            bad.append(key)
            continue
        # The reference path sums in float32, the oracle in float64: a finite
        # page may swap with a near-tied one (the gap rule), nothing else.
        only_w = sorted(set(ids_w) - set(ids_r))
        only_r = sorted(set(ids_r) - set(ids_w))
        row = scores[key[0], key[1]]
        for a, c in zip(only_w, only_r):
            sa, sc = float(row[a]), float(row[c])
            if not (math.isfinite(sa) and math.isfinite(sc) and abs(sa - sc) <= 1e-4 * abs(sa)):
                bad.append(key)
        if len(only_w) != len(only_r):
            bad.append(key)
    assert not bad, [(key, got_w[key], got_r[key]) for key in bad[:4]]
    # The rule is exercised: NaN picks became -1 and some rows lost forced pages.
    # Row 900 (page 14): eleven NaN pages outrank the four forced ones, so every
    # slot is a NaN pick.
    assert got_w[1, 900] == ([], want.shape[-1])
    assert any(n > 0 and ids for (ids, n) in got_w.values())
    n_nan_rows = sum(1 for r in special for g in range(2) if bool(torch.isnan(scores[g, r]).any()))
    assert n_nan_rows >= 4


def test_a_planted_nan_ordering_mistake_is_caught(monkeypatch):
    case, q, k = _planted_case()
    real = leanselect_oracle._stable_topk_desc

    def nan_last(scores, kk):  # the mistake: NaN ranked below every number
        return real(torch.where(torch.isnan(scores), torch.full_like(scores, -math.inf),
                                scores), kk)

    monkeypatch.setattr(leanselect_oracle, "_stable_topk_desc", nan_last)
    want, ref, _ = _plans(case, q, k)
    rows = [800, 850, 900, 950, 64 * 3 + 40, 600]
    got_w, got_r = _rows_as_sets(want, rows), _rows_as_sets(ref, rows)
    assert any(got_w[key] != got_r[key] for key in got_w)


@pytest.mark.parametrize("vals, k, want", [
    ([1.0, float("nan"), float("inf"), 2.0], 2, [1, 2]),
    ([float("nan"), float("nan"), 0.0], 1, [0]),
    ([float("-inf"), 3.0, 3.0, float("nan")], 3, [3, 1, 2]),
])
def test_stable_topk_ranks_nan_first_like_torch_sort(vals, k, want):
    x = torch.tensor(vals, dtype=torch.float64)
    got = leanselect_oracle._stable_topk_desc(x, k).tolist()
    assert got == want
    # torch's stable descending sort puts NaN first and keeps ties in index order.
    assert got == torch.sort(x, descending=True, stable=True).indices[:k].tolist()
