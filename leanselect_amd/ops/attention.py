"""Block-sparse prefill attention on the GPU.

``infllmv2_attn_varlen_func`` keeps the call surface the reference's model files
use (leanselect/models/minicpm.py:3229-3243; nosa.py:2220-2251; wrapper contract
third_party/infllmv2/paper1.patch:1993-2100) and runs ``ls_sparse_attn_varlen``.
"""
from __future__ import annotations

import torch

from .. import _hip

__all__ = ["attention_tile_rows", "infllmv2_attn_varlen_func", "sparse_attention"]

def attention_tile_rows(take: int) -> int:
    """Query rows per workgroup of the attention kernel for plans of ``take`` ids a
    row: 24 (three rows per wave) for every width it accepts (at most 128 ids; the
    union of a tile, at most 3072 pages, fits its 4096-entry table), as the launcher
    in csrc/ls_attention.hip uses."""
    if take > 128:
        raise ValueError("the attention kernel accepts at most 128 ids per row")
    return 24


def sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    topk_idx: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    causal: bool = True,
    block_size: int = 64,
    return_lse: bool = False,
    out: torch.Tensor | None = None,
    sync_status: bool = False,
):
    """``out [total_q, H, D]`` (and ``lse [H, total_q]`` float32 with ``return_lse``).

    The kernel reports an expired wait for a staged page in a status word (and
    writes the affected rows as NaN).  The word is checked without stalling the
    host: an expired wait raises ``RuntimeError`` at a later attention call or
    at ``leanselect_amd._hip.attn_status_sync()``; ``sync_status=True`` waits
    for this call and raises at once."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k, v must be [tokens, heads, head_dim]")
    if topk_idx is None or topk_idx.ndim != 3:
        raise ValueError("topk_idx must be [num_kv_heads, total_q, k] int32")
    # Host-side checks first: no launch may see int64 offsets or a misshapen output.
    _hip.check_cu_seqlens(cu_seqlens_q, cu_seqlens_k)
    if out is not None:
        _hip.check_out(out, tuple(q.shape), q.dtype, q.device)
    dev = _hip.require_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k, topk_idx)
    total_q, H, D = q.shape
    total_k, G, Dk = k.shape
    if v.shape != k.shape or Dk != D:
        raise ValueError("k and v must be [total_k, num_kv_heads, head_dim] like q's head_dim")
    if H % G:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if topk_idx.shape[0] != G or topk_idx.shape[1] != total_q:
        raise ValueError(f"topk_idx must be [{G}, {total_q}, k], got {tuple(topk_idx.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k and v must share a dtype")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("sparse attention supports fp16 and bf16 only")
    if topk_idx.dtype != torch.int32:
        topk_idx = topk_idx.to(torch.int32)
    q = q if (q.stride(2) == 1 and q.stride(1) == D) else q.contiguous()
    k = k if (k.stride(2) == 1 and k.stride(1) == D) else k.contiguous()
    v = v if (v.stride(2) == 1 and v.stride(1) == D) else v.contiguous()
    topk_idx = topk_idx.contiguous()
    batch = cu_seqlens_q.numel() - 1
    if out is None:
        out = torch.empty((total_q, H, D), dtype=q.dtype, device=dev)
    lse = torch.empty((H, total_q), dtype=torch.float32, device=dev) if return_lse else None
    L = _hip.lib()
    dt = _hip.dtype_code(q.dtype)
    ws = _hip.workspace(L.ls_sparse_attn_workspace_size(total_k, batch, G, D, int(max_seqlen_k), dt), dev)
    scale = -1.0 if softmax_scale is None else float(softmax_scale)
    rc = L.ls_sparse_attn_varlen(
        q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
        cu_seqlens_q.contiguous().data_ptr(), cu_seqlens_k.contiguous().data_ptr(), batch,
        total_q, total_k, int(max_seqlen_q), int(max_seqlen_k), H, G, D, dt,
        topk_idx.data_ptr(), topk_idx.shape[2], block_size, scale, 1 if causal else 0,
        out.data_ptr(), _hip.ptr(lse), ws.data_ptr(), ws.numel(), _hip.stream_of(dev))
    _hip.check(rc, "ls_sparse_attn_varlen")
    if total_q > 0 and batch > 0:  # an empty call launches nothing and leaves no status
        _hip.check_attn_status(ws, "ls_sparse_attn_varlen", sync=sync_status)
    return (out, lse) if return_lse else out


def infllmv2_attn_varlen_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    dropout_p: float = 0.0,
    softmax_scale: float | None = None,
    causal: bool = False,
    window_size=(-1, -1),
    softcap: float = 0.0,
    alibi_slopes=None,
    deterministic: bool = False,
    return_attn_probs: bool = False,
    block_table=None,
    topk_idx: torch.Tensor | None = None,
):
    """Sparse varlen attention with the InfLLM-v2 call surface.

    Returns ``out`` or, with ``return_attn_probs``, ``(out, softmax_lse, S_dmask)``
    where ``softmax_lse`` is ``[H, total_q]`` float32 and ``S_dmask`` is empty
    (inference: no dropout mask).  Only the sparse path (``topk_idx`` given,
    no dropout, no window/softcap/alibi/paged KV) is provided.
    """
    if topk_idx is None:
        raise NotImplementedError("only the block-sparse path (topk_idx=...) is provided")
    if dropout_p:
        raise NotImplementedError("dropout is not supported (prefill inference)")
    if tuple(window_size) != (-1, -1) or softcap or alibi_slopes is not None or block_table is not None:
        raise NotImplementedError("window_size / softcap / alibi / block_table are not supported")
    del deterministic
    res = sparse_attention(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, topk_idx,
        softmax_scale=softmax_scale, causal=causal, return_lse=return_attn_probs)
    if return_attn_probs:
        out, lse = res
        return out, lse, torch.empty(0, dtype=q.dtype, device=q.device)
    return res
