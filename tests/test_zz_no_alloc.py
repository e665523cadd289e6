"""The allocation-free attention entry point (``ls_sparse_attn_varlen_noalloc``)
against ``ls_sparse_attn_varlen`` through the C ABI: identical outputs on two
calls in a row (the second on a smaller batch, so stale contents of the
shared static scratch would show), and oversized requests rejected before any
device work."""
import ctypes

import pytest
import torch

from leanselect_amd import _hip, workloads
from leanselect_amd.ops import compress_k, leanselect_prefill_topk_idx, sparse_attention


def _case(lens, seed):
    case = workloads.hidden_space_layer(lens, hidden=1024, device="cuda", seed=seed)
    kc, cu_c = compress_k(case.k, case.cu_seqlens, cu_seqlens_host=case.cu_host)
    ids = leanselect_prefill_topk_idx(case.q, kc, case.cu_seqlens, cu_c, case.selector,
                                      topk=case.topk, init_blocks=case.init_blocks,
                                      local_blocks=case.local_blocks,
                                      cu_seqlens_q_host=case.cu_host)
    return case, ids


def _noalloc(case, ids, out, lse, status):
    L = _hip.lib()
    total, H, D = case.q.shape
    G = case.k.shape[1]
    rc = L.ls_sparse_attn_varlen_noalloc(
        case.q.data_ptr(), case.q.stride(0), case.k.data_ptr(), case.k.stride(0),
        case.v.data_ptr(), case.v.stride(0), case.cu_seqlens.data_ptr(),
        case.cu_seqlens.data_ptr(), len(case.cu_host) - 1, total, total, case.max_seqlen,
        case.max_seqlen, H, G, D, _hip.LS_BF16, ids.data_ptr(), ids.shape[2], 64, -1.0, 1,
        out.data_ptr(), lse.data_ptr(), status.data_ptr(), _hip.stream_of(out.device))
    _hip.check(rc, "ls_sparse_attn_varlen_noalloc")


@pytest.mark.gpu
def test_noalloc_matches_the_workspace_entry_point():
    for lens, seed in (((3000, 1500), 41), ((700,), 42)):  # the second call is smaller
        case, ids = _case(lens, seed)
        want, want_lse = sparse_attention(case.q, case.k, case.v, case.cu_seqlens,
                                          case.cu_seqlens, case.max_seqlen, case.max_seqlen, ids,
                                          return_lse=True)
        out = torch.full_like(want, float("nan"))
        lse = torch.full_like(want_lse, float("nan"))
        status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        _noalloc(case, ids, out, lse, status)
        torch.cuda.synchronize()
        print(f"\nnoalloc {lens}: status {int(status.item())}", flush=True)
        assert int(status.item()) == 0
        assert torch.equal(out, want)
        assert torch.equal(lse, want_lse)


@pytest.mark.gpu
def test_noalloc_empty_call_writes_a_clean_status():
    """A call with no query rows launches no attention kernel; the caller's
    status word (pre-filled with -1 here) is still written with 0."""
    L = _hip.lib()
    G, H, D = 2, 8, 128
    q = torch.empty(0, H, D, dtype=torch.bfloat16, device="cuda")
    k = torch.randn(128, G, D, device="cuda").to(torch.bfloat16)
    cu_q = torch.zeros(2, dtype=torch.int32, device="cuda")
    cu_k = torch.tensor([0, 128], dtype=torch.int32, device="cuda")
    ids = torch.empty(G, 0, 4, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    rc = L.ls_sparse_attn_varlen_noalloc(
        q.data_ptr(), H * D, k.data_ptr(), G * D, k.data_ptr(), G * D, cu_q.data_ptr(),
        cu_k.data_ptr(), 1, 0, 128, 0, 128, H, G, D, _hip.LS_BF16, ids.data_ptr(), 4, 64, -1.0,
        1, out.data_ptr(), None, status.data_ptr(), _hip.stream_of(q.device))
    _hip.check(rc, "ls_sparse_attn_varlen_noalloc")
    torch.cuda.synchronize()
    assert int(status.item()) == 0


def test_noalloc_rejects_requests_above_the_static_scratch():
    # 2 KV heads x 1100 pages of staged K/V exceed 64 MiB; nothing is dereferenced
    # and no device is touched before the size check.
    L = _hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    rc = L.ls_sparse_attn_varlen_noalloc(
        fake, 4096, fake, 256, fake, 256, fake, fake, 1, 70000, 70000, 70000, 70000, 32, 2, 128,
        _hip.LS_BF16, fake, 64, 64, -1.0, 1, fake, None, None, None)
    assert rc == _hip.LS_ERR_UNSUPPORTED
    assert b"static" in L.ls_last_error()
