"""Prefill page selection on the GPU.

Mirrors the LeanSelect branch of
``MiniCPMInfLLMv2Attention._lightweight_compressed_attention``
(leanselect/models/minicpm.py:3061-3142): one page plan per KV group and query
token, ``take = min(topk, max_pages)`` slots, sink and local pages forced,
invisible pages never chosen, ``-1`` padding.  The whole chain (router
projection, atom scores, 5-atom page max, forcing, top-k) runs in
``ls_select_prefill``; rows list their ids in ascending order.
"""
from __future__ import annotations

import torch

from .. import _hip

__all__ = ["leanselect_prefill_topk_idx", "select_take"]


def select_take(cu_seqlens_q_host: list[int], topk: int, block_size: int) -> int:
    """``min(topk, max_pages)`` over the packed sequences (minicpm.py:3096-3104)."""
    max_pages = max(
        ((cu_seqlens_q_host[b + 1] - cu_seqlens_q_host[b] + block_size - 1) // block_size
         for b in range(len(cu_seqlens_q_host) - 1)),
        default=0,
    )
    return min(int(topk), max_pages)


def _masters(selector) -> list[torch.Tensor]:
    out = []
    for name in ("head_mix", "kv_head_mix", "q_proj", "k_proj"):
        t = getattr(selector, name).detach()
        if t.dtype != torch.float32:
            t = t.float()
        out.append(t.contiguous())
    return out


def leanselect_prefill_topk_idx(
    q_unpad: torch.Tensor,
    k_compressed: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    selector,
    *,
    topk: int,
    block_size: int = 64,
    kernel_stride: int = 16,
    init_blocks: int = 1,
    local_blocks: int = 32,
    cache_lens: torch.Tensor | None = None,
    cu_seqlens_q_host: list[int] | None = None,
    q_tilde: torch.Tensor | None = None,
) -> torch.Tensor:
    """Page plans ``topk_idx [G, total_q, take]`` int32.

    ``q_unpad [total_q, H, D]`` are the post-RoPE queries, ``k_compressed
    [total_atoms, G, D]`` the compressed keys with prefix offsets
    ``cu_seqlens_k`` (int32, device), ``selector`` a ``LeanSelectSelector``.
    ``q_tilde [G, total_q, R*F]``, when given, is the selector's projection of
    those queries (as ``rope_project_queries`` forms it while rotating them);
    the selection then does not read ``q_unpad``.
    """
    if cache_lens is not None:
        raise ValueError("Lightweight selection is prefill only")
    if q_unpad.ndim != 3 or k_compressed.ndim != 3:
        raise ValueError("q_unpad must be [total_q, H, D] and k_compressed [A, G, D]")
    dev = _hip.require_gpu(q_unpad, k_compressed, cu_seqlens_q, cu_seqlens_k)
    if cu_seqlens_q.dtype != torch.int32 or cu_seqlens_k.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32")
    if q_unpad.dtype != k_compressed.dtype:
        raise ValueError("q_unpad and k_compressed must share a dtype")
    total_q, H, D = q_unpad.shape
    G = k_compressed.shape[1]
    if (H, G, D) != (selector.num_heads, selector.num_kv_heads, selector.head_dim):
        raise ValueError("query / compressed-key shapes do not match the selector")
    if q_unpad.stride(2) != 1 or q_unpad.stride(1) != D:
        q_unpad = q_unpad.contiguous()
    if k_compressed.stride(2) != 1 or k_compressed.stride(1) != D:
        k_compressed = k_compressed.contiguous()
    host = cu_seqlens_q_host if cu_seqlens_q_host is not None else cu_seqlens_q.tolist()
    batch = len(host) - 1
    max_seqlen_q = max((host[b + 1] - host[b] for b in range(batch)), default=0)
    take = select_take(host, topk, block_size)
    if take == 0 or total_q == 0:
        return torch.full((G, total_q, take), -1, dtype=torch.int32, device=dev)
    # Every slot of every row is written by the kernel.
    topk_idx = torch.empty((G, total_q, take), dtype=torch.int32, device=dev)
    dt = _hip.dtype_code(q_unpad.dtype)
    hm, khm, qp, kp = _masters(selector)
    L = _hip.lib()
    total_atoms = k_compressed.shape[0]
    max_pages = (max_seqlen_q + block_size - 1) // block_size
    nbytes = L.ls_select_workspace_size(
        total_q, total_atoms, batch, H, G, D, selector.router_heads, selector.router_dim,
        max_pages, dt)
    ws = _hip.workspace(nbytes, dev)
    if q_tilde is not None:
        F = selector.router_heads * selector.router_dim
        if tuple(q_tilde.shape) != (G, total_q, F) or q_tilde.dtype != q_unpad.dtype \
                or not q_tilde.is_contiguous() or q_tilde.device != q_unpad.device:
            raise ValueError(f"q_tilde must be a contiguous [{G}, {total_q}, {F}] "
                             f"{q_unpad.dtype} tensor on {q_unpad.device}")
        rc = L.ls_select_prefill_qt(
            q_tilde.data_ptr(), total_q,
            k_compressed.data_ptr() if total_atoms else None, k_compressed.stride(0), total_atoms,
            cu_seqlens_q.contiguous().data_ptr(), cu_seqlens_k.contiguous().data_ptr(), batch,
            max_seqlen_q, H, G, D, khm.data_ptr(), kp.data_ptr(), selector.router_heads,
            selector.router_dim, dt, int(topk), block_size, kernel_stride, int(init_blocks),
            int(local_blocks), topk_idx.data_ptr(), take, ws.data_ptr(), ws.numel(),
            _hip.stream_of(dev))
        _hip.check(rc, "ls_select_prefill_qt")
        return topk_idx
    rc = L.ls_select_prefill(
        q_unpad.data_ptr(), q_unpad.stride(0), total_q,
        k_compressed.data_ptr() if total_atoms else None, k_compressed.stride(0), total_atoms,
        cu_seqlens_q.contiguous().data_ptr(), cu_seqlens_k.contiguous().data_ptr(), batch,
        max_seqlen_q, H, G, D, hm.data_ptr(), khm.data_ptr(), qp.data_ptr(), kp.data_ptr(),
        selector.router_heads, selector.router_dim, dt, int(topk), block_size, kernel_stride,
        int(init_blocks), int(local_blocks), topk_idx.data_ptr(), take, ws.data_ptr(),
        ws.numel(), _hip.stream_of(dev))
    _hip.check(rc, "ls_select_prefill")
    return topk_idx
