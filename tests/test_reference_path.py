"""The CPU baseline's restatement of the reference's own torch formulation
(activation-dtype einsums, max_pool1d, torch.topk) agrees with the float64
oracle: page plans under the north-star gap rule, compressed keys and attention
within float32 accumulation error."""
import torch

import oracle
from leanselect_amd import workloads


def _masters(sel):
    return [getattr(sel, n).detach().float() for n in ("head_mix", "kv_head_mix", "q_proj", "k_proj")]


def _compare(case, dtype):
    cu = case.cu_host
    kc, cu_c = oracle.reference_compress_k(case.k, cu)
    want_kc, want_cu = oracle.compress_k(case.k, cu)
    assert cu_c == want_cu.tolist()
    torch.testing.assert_close(kc.double(), want_kc.double(), rtol=1e-2 if dtype != torch.float32 else 1e-6,
                               atol=1e-2 if dtype != torch.float32 else 1e-6)
    ids = oracle.reference_select_prefill(case.q, want_kc, cu, want_cu.tolist(), _masters(case.selector),
                                          topk=case.topk, init_blocks=case.init_blocks,
                                          local_blocks=case.local_blocks)
    qf, kf = oracle.fused_weights(*_masters(case.selector), dtype)
    rows = list(range(0, cu[-1], 3))
    want, scores = oracle.select_prefill(case.q, want_kc, cu, want_cu.tolist(), qf, kf,
                                         topk=case.topk, init_blocks=case.init_blocks,
                                         local_blocks=case.local_blocks, rows=rows,
                                         return_scores=True)
    got = torch.sort(ids[:, rows].long().masked_fill(ids[:, rows] < 0, 1 << 20), -1).values
    got = got.masked_fill(got == 1 << 20, -1).to(torch.int32)
    return oracle.check_topk(got, want, scores, dtype)


def test_reference_path_selection_fp32():
    case = workloads.head_space_layer(2048, seed=3)
    rep = _compare(case, torch.float32)
    assert rep.ok, str(rep)
    assert rep.exact_rows >= 0.99 * rep.rows


def test_reference_path_selection_bf16_ragged():
    case = workloads.hidden_space_layer((700, 1500), hidden=512, seed=4)
    rep = _compare(case, torch.bfloat16)
    # The reference's bf16 einsums round each contraction's float32 partial
    # sums differently from the oracle's single rounding of a float64 sum, so a
    # boundary page can move by a quantisation step on a few rows; the plans
    # agree on the rest.
    print(rep)
    assert rep.exact_rows >= 0.9 * rep.rows


def test_reference_path_attention_matches_oracle():
    case = workloads.head_space_layer(1024, seed=5)
    qf, kf = oracle.fused_weights(*_masters(case.selector), torch.float32)
    kc, cu_c = oracle.compress_k(case.k, case.cu_host)
    ids = oracle.select_prefill(case.q, kc, case.cu_host, cu_c.tolist(), qf, kf, topk=case.topk,
                                init_blocks=case.init_blocks, local_blocks=case.local_blocks)
    rows = list(range(0, 1024, 37)) + [1023]
    got = oracle.reference_sparse_attention_rows(case.q, case.k, case.v, case.cu_host, ids, rows)
    want, _ = oracle.sparse_attention(case.q, case.k, case.v, case.cu_host, case.cu_host, ids,
                                      rows=rows)
    torch.testing.assert_close(got.double(), want.double(), rtol=1e-4, atol=1e-5)
