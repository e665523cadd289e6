"""Selection with NaN and infinite scores against the oracle (the reference's
rule, leanselect/models/minicpm.py:3124-3141): visible pages ranked with forced
pages at +inf, torch.topk ranking NaN above +inf, and the chosen pages with a
NaN or -inf score emitted as -1.

NaN and +-inf are planted in query rows (a query row's q~ becomes NaN or mixed
+-inf for its KV group, so every non-forced page of that row scores NaN) and in
key rows (the compressed windows holding them, and so the pages around them,
score NaN for every later row).  Rows with more NaN pages than their budget
lose their forced pages as well; small budgets (fewer slots than forced pages)
take the path that never ranks the other pages.  Every sampled row must give
exactly the oracle's set of valid ids."""
import dataclasses

import pytest
import torch

from gpu_helpers import oracle_select_rows, spread_rows
from leanselect_amd import workloads
from leanselect_amd.ops import compress_k, leanselect_prefill_topk_idx

pytestmark = pytest.mark.gpu
DEV = "cuda"


NEG_NAN = "-nan"  # a NaN with the sign bit set (Python's -nan keeps a positive sign in torch)
_NEG_NAN_BITS = {torch.bfloat16: (torch.int16, -64), torch.float16: (torch.int16, -512),
                 torch.float32: (torch.int32, -4194304)}  # 0xffc0, 0xfe00, 0xffc00000


def _set(t, idx, val):
    if val == NEG_NAN:
        it, bits = _NEG_NAN_BITS[t.dtype]
        t.view(it)[idx] = bits
        assert bool(torch.isnan(t[idx].float()))
    else:
        t[idx] = val


def _plant(case, q_cells, k_cells):
    q = case.q.clone()
    k = case.k.clone()
    for idx, val in q_cells:
        _set(q, idx, val)
    for idx, val in k_cells:
        _set(k, idx, val)
    return dataclasses.replace(case, q=q, k=k)


def _compare(case, topk, rows):
    kc, cu_c = compress_k(case.k, case.cu_seqlens, cu_seqlens_host=case.cu_host)
    ids = leanselect_prefill_topk_idx(
        case.q, kc, case.cu_seqlens, cu_c, case.selector, topk=topk,
        init_blocks=case.init_blocks, local_blocks=case.local_blocks,
        cu_seqlens_q_host=case.cu_host)
    c2 = dataclasses.replace(case, topk=topk)
    want, scores = oracle_select_rows(c2, kc.cpu(), cu_c.cpu().tolist(), rows, case.q.dtype)
    got = ids.cpu()[:, rows]
    bad, n_invalid, n_nan_rows = [], 0, 0
    for g in range(got.shape[0]):
        for i, r in enumerate(rows):
            a = sorted(int(x) for x in got[g, i] if x >= 0)
            b = sorted(int(x) for x in want[g, i] if x >= 0)
            n_invalid += int((got[g, i] < 0).sum())
            n_nan_rows += int(torch.isnan(scores[g, i]).any())
            if a != b or int((got[g, i] < 0).sum()) != int((want[g, i] < 0).sum()):
                bad.append((g, r, a[:8], b[:8]))
    print(f"\nNaN/inf selection topk={topk}: rows={len(rows)} x {got.shape[0]} groups, "
          f"rows with NaN scores={n_nan_rows}, -1 slots={n_invalid}, mismatches={len(bad)} "
          f"first={bad[:3]}", flush=True)
    assert not bad
    return n_nan_rows


@pytest.mark.parametrize("topk", [64, 4])
def test_nan_and_inf_in_queries_and_keys_bf16(topk):
    case = workloads.hidden_space_layer((8192,), hidden=1024, device=DEV, seed=31)
    nan, inf = float("nan"), float("inf")
    q_rows = [100, 2600, 4000, 6500, 8191, 1234, 7000]
    q_cells = [((100, 3, 5), nan), ((2600, 3, 5), nan), ((4000, 20, 9), nan),
               ((6500, 3, 5), NEG_NAN), ((8191, 1, 0), nan), ((1234, 20, 7), inf),
               ((7000, 5, 77), -inf)]
    k_cells = [((64 * 37 + 5, 1, 9), nan), ((64 * 90 + 40, 0, 2), inf),
               ((64 * 110 + 3, 0, 4), NEG_NAN)]
    case = _plant(case, q_cells, k_cells)
    rows = sorted(set(spread_rows(case.cu_host, per_seq=48)) | set(q_rows) |
                  {64 * 38 + 7, 64 * 40, 64 * 95, 64 * 115 + 1})
    assert _compare(case, topk, rows) > 0


def test_nan_in_queries_fp32():
    """The float32 path (32-bit keys): the CPU-runnable layer with NaN query rows."""
    case = workloads.head_space_layer(4096, device=DEV)
    nan = float("nan")
    q_rows = [70, 1500, 4000]
    case = _plant(case, [((r, 2, 3), nan) for r in q_rows] + [((2222, 6, 1), NEG_NAN)],
                  [((64 * 20 + 1, 0, 0), nan)])
    rows = sorted(set(spread_rows(case.cu_host, per_seq=48)) | set(q_rows) | {2222})
    assert _compare(case, case.topk, rows) > 0
