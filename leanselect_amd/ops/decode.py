"""Decode over a KV cache on the GPU.

Three operators, each one C-ABI call:

- ``kvcache_append``: packed new keys/values into a padded per-sequence cache,
  plus the compressed key windows the new tokens complete
  (``InfLLMv2CacheLayer.update`` / ``update_no_compress_k`` / ``update_compress_k``,
  leanselect/models/minicpm.py:1237-1325, 2888-2958);
- ``decode_topk_idx``: stage-1 page plans of decode rows
  (``compressed_attention`` with ``cache_lens``, minicpm.py:594-705);
- ``sparse_attention_kvcache``: block-sparse attention of the rows over the
  cache (``infllmv2_attn_with_kvcache(..., topk_idx=)``,
  third_party/infllmv2/paper1.patch:2511-2615).

The cache layout is ``[batch, capacity, num_kv_heads, head_dim]`` per tensor;
``capacity`` is a multiple of the 64-token page.
"""
from __future__ import annotations

import torch

from .. import _hip

__all__ = ["n_windows", "kvcache_append", "decode_topk_idx", "sparse_attention_kvcache",
           "decode_out_len", "stage1_scores"]


def n_windows(length: int, kernel_size: int = 32, kernel_stride: int = 16) -> int:
    """Compressed windows of a ``length``-token sequence."""
    return (length - kernel_size) // kernel_stride + 1 if length >= kernel_size else 0


def _lengths(t: torch.Tensor, host, name: str) -> list[int]:
    if t.dtype != torch.int32 or t.ndim != 1:
        raise ValueError(f"{name} must be a 1-D int32 tensor")
    return [int(x) for x in (host if host is not None else t.tolist())]


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if k_cache.ndim != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache must be [batch, capacity, num_kv_heads, head_dim]")
    if k_cache.dtype != v_cache.dtype or k_cache.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("the cache must be bf16 or fp16, k and v alike")
    D = k_cache.shape[3]
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        if t.stride(3) != 1 or t.stride(2) != D or t.stride(0) != k_cache.stride(0) \
                or t.stride(1) != k_cache.stride(1):
            raise ValueError(f"{name} must have dense [num_kv_heads, head_dim] rows and the "
                             "same strides as the other cache tensor")


def kvcache_append(k_cache: torch.Tensor, v_cache: torch.Tensor, cache_seqlens: torch.Tensor,
                   k_new: torch.Tensor, v_new: torch.Tensor, cu_seqlens_new: torch.Tensor, *,
                   kc_cache: torch.Tensor | None = None, kernel_size: int = 32,
                   kernel_stride: int = 16, cache_seqlens_host: list[int] | None = None,
                   cu_seqlens_new_host: list[int] | None = None) -> None:
    """Write ``k_new / v_new [total_new, G, D]`` (sequence ``b``'s rows are
    ``cu_seqlens_new[b]:cu_seqlens_new[b+1]``) at positions ``cache_seqlens[b] + i``
    and, with ``kc_cache [batch, kc_capacity, G, D]``, the compressed windows the
    new tokens complete.  ``cache_seqlens`` is left as it is (advance it after)."""
    _check_cache(k_cache, v_cache)
    if k_new.ndim != 3 or v_new.shape != k_new.shape:
        raise ValueError("k_new and v_new must be [total_new, num_kv_heads, head_dim]")
    B, cap, G, D = k_cache.shape
    if tuple(k_new.shape[1:]) != (G, D) or k_new.dtype != k_cache.dtype or v_new.dtype != k_cache.dtype:
        raise ValueError("new keys/values must match the cache's heads, head_dim and dtype")
    lens = _lengths(cache_seqlens, cache_seqlens_host, "cache_seqlens")
    cu = _lengths(cu_seqlens_new, cu_seqlens_new_host, "cu_seqlens_new")
    if len(lens) != B or len(cu) != B + 1 or cu[0] != 0 or cu[-1] != k_new.shape[0] \
            or any(cu[b + 1] < cu[b] for b in range(B)):
        raise ValueError("cache_seqlens must be [batch] and cu_seqlens_new [batch + 1] offsets "
                         "of the packed new rows")
    n_new = [cu[b + 1] - cu[b] for b in range(B)]
    if any(lens[b] < 0 or lens[b] + n_new[b] > cap for b in range(B)):
        raise ValueError(f"appending {n_new} tokens to {lens} exceeds the capacity {cap}")
    new_windows = 0
    if kc_cache is not None:
        if kc_cache.ndim != 4 or kc_cache.shape[0] != B or tuple(kc_cache.shape[2:]) != (G, D) \
                or kc_cache.dtype != k_cache.dtype or kc_cache.stride(3) != 1 \
                or kc_cache.stride(2) != D:
            raise ValueError("kc_cache must be [batch, kc_capacity, num_kv_heads, head_dim] "
                             "like the cache")
        for b in range(B):
            nw = n_windows(lens[b] + n_new[b], kernel_size, kernel_stride)
            if nw > kc_cache.shape[1]:
                raise ValueError(f"{nw} compressed windows exceed kc_capacity {kc_cache.shape[1]}")
            new_windows += nw - n_windows(lens[b], kernel_size, kernel_stride)
    dev = _hip.require_gpu(k_cache, v_cache, cache_seqlens, k_new, v_new, cu_seqlens_new, kc_cache)
    # One row stride serves both: dense rows with equal strides, else copies.
    if not (k_new.stride(2) == 1 and k_new.stride(1) == D and v_new.stride() == k_new.stride()
            and k_new.stride(0) % 8 == 0):
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    cu_win = torch.empty(B + 1, dtype=torch.int32, device=dev) if kc_cache is not None else None
    rc = _hip.lib().ls_kvcache_append(
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        cache_seqlens.contiguous().data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0),
        cu_seqlens_new.contiguous().data_ptr(), k_new.shape[0], B, G, D,
        _hip.dtype_code(k_cache.dtype), _hip.ptr(kc_cache),
        kc_cache.stride(0) if kc_cache is not None else 0,
        kc_cache.stride(1) if kc_cache is not None else 0, new_windows, int(kernel_size),
        int(kernel_stride), _hip.ptr(cu_win), _hip.stream_of(dev))
    _hip.check(rc, "ls_kvcache_append")


def decode_out_len(seqlens_k: list[int], len_q: list[int], block_size: int = 64) -> int:
    """Pooled page columns: ``ceil((max len_q + max(len_k - len_q)) / block_size)``
    (``max_pooling_1d_varlen``'s ``out_len`` with ``cache_lens = len_k - len_q``)."""
    if not seqlens_k:
        return 0
    return (max(len_q) + max(k - q for k, q in zip(seqlens_k, len_q)) + block_size - 1) // block_size


def decode_topk_idx(q: torch.Tensor, kc_cache: torch.Tensor, cache_seqlens: torch.Tensor,
                    cu_seqlens_q: torch.Tensor, *, topk: int, init_blocks: int = 1,
                    local_blocks: int = 32, block_size: int = 64, kernel_size: int = 32,
                    kernel_stride: int = 16, softmax_scale: float | None = None,
                    cache_seqlens_host: list[int] | None = None,
                    cu_seqlens_q_host: list[int] | None = None) -> torch.Tensor:
    """Stage-1 page plans ``[G, total_q, min(topk, out_len)]`` int32 of the query
    rows ``q [total_q, H, D]`` (row ``i`` of sequence ``b`` at position
    ``cache_seqlens[b] - len_q(b) + i``; ``cache_seqlens`` already counts the
    rows' tokens) over the compressed-key cache ``kc_cache [batch, kc_capacity, G, D]``."""
    if q.ndim != 3 or kc_cache.ndim != 4:
        raise ValueError("q must be [total_q, H, D] and kc_cache [batch, kc_capacity, G, D]")
    total_q, H, D = q.shape
    B, _, G, Dk = kc_cache.shape
    if Dk != D or H % G or q.dtype != kc_cache.dtype:
        raise ValueError("q and kc_cache must share head_dim and dtype, H divisible by G")
    lens = _lengths(cache_seqlens, cache_seqlens_host, "cache_seqlens")
    cu = _lengths(cu_seqlens_q, cu_seqlens_q_host, "cu_seqlens_q")
    if len(lens) != B or len(cu) != B + 1 or cu[0] != 0 or cu[-1] != total_q:
        raise ValueError("cache_seqlens must be [batch] and cu_seqlens_q [batch + 1] offsets of q")
    len_q = [cu[b + 1] - cu[b] for b in range(B)]
    if any(len_q[b] < 0 or len_q[b] > lens[b] for b in range(B)):
        raise ValueError("every sequence must hold its query rows (0 <= len_q <= cache length)")
    if kc_cache.stride(3) != 1 or kc_cache.stride(2) != D or kc_cache.stride(1) != G * D:
        raise ValueError("kc_cache rows must be dense")
    max_kc = max(n_windows(x, kernel_size, kernel_stride) for x in lens)
    if max_kc > kc_cache.shape[1]:
        raise ValueError("kc_cache holds fewer windows than the sequences have")
    out_len = decode_out_len(lens, len_q, block_size)
    take = min(int(topk), out_len)
    dev = _hip.require_gpu(q, kc_cache, cache_seqlens, cu_seqlens_q)
    if total_q == 0 or take <= 0:
        return torch.full((G, total_q, max(take, 0)), -1, dtype=torch.int32, device=dev)
    q = q if (q.stride(2) == 1 and q.stride(1) == D) else q.contiguous()
    L = _hip.lib()
    ws = _hip.workspace(L.ls_decode_select_workspace_size(total_q, B, G, max_kc, out_len), dev)
    ids = torch.empty((G, total_q, take), dtype=torch.int32, device=dev)
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    rc = L.ls_decode_select(
        q.data_ptr(), q.stride(0), cu_seqlens_q.contiguous().data_ptr(), total_q,
        kc_cache.data_ptr(), kc_cache.stride(0), kc_cache.stride(1),
        cache_seqlens.contiguous().data_ptr(), B, max_kc, H, G, D, _hip.dtype_code(q.dtype), scale,
        int(topk), int(block_size), int(kernel_size), int(kernel_stride), int(init_blocks),
        int(local_blocks), out_len, take, ids.data_ptr(), ws.data_ptr(), ws.numel(),
        _hip.stream_of(dev))
    _hip.check(rc, "ls_decode_select")
    return ids


def sparse_attention_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             cache_seqlens: torch.Tensor, topk_idx: torch.Tensor,
                             cu_seqlens_q: torch.Tensor, *, causal: bool = False,
                             softmax_scale: float | None = None, n_splits: int | None = None,
                             return_lse: bool = False, out: torch.Tensor | None = None):
    """``out [total_q, H, D]`` of the rows ``q [total_q, H, D]`` over the cache,
    restricted to each row's plan ``topk_idx [G, total_q, k]`` (and ``lse [H,
    total_q]`` float32 with ``return_lse``)."""
    _check_cache(k_cache, v_cache)
    if q.ndim != 3 or topk_idx is None or topk_idx.ndim != 3:
        raise ValueError("q must be [total_q, H, D] and topk_idx [G, total_q, k]")
    total_q, H, D = q.shape
    B, cap, G, Dk = k_cache.shape
    if Dk != D or H % G or q.dtype != k_cache.dtype:
        raise ValueError("q and the cache must share head_dim and dtype, H divisible by G")
    if topk_idx.shape[0] != G or topk_idx.shape[1] != total_q or not 1 <= topk_idx.shape[2] <= 256:
        raise ValueError(f"topk_idx must be [{G}, {total_q}, k] with 1 <= k <= 256")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.numel() != B \
            or cu_seqlens_q.dtype != torch.int32 or cu_seqlens_q.numel() != B + 1:
        raise ValueError("cache_seqlens must be int32 [batch] and cu_seqlens_q int32 [batch + 1]")
    if out is not None:
        _hip.check_out(out, (total_q, H, D), q.dtype, q.device)
    dev = _hip.require_gpu(q, k_cache, v_cache, cache_seqlens, topk_idx, cu_seqlens_q)
    if topk_idx.dtype != torch.int32:
        topk_idx = topk_idx.to(torch.int32)
    topk_idx = topk_idx.contiguous()
    q = q if (q.stride(2) == 1 and q.stride(1) == D) else q.contiguous()
    K = topk_idx.shape[2]
    if n_splits is None:
        # Workgroups of four waves per (row, group): enough of them to cover the
        # device when there are few rows, at least one page per wave.
        n_splits = max(1, min(-(-K // 4), -(-256 // max(1, total_q * G))))
    n_splits = max(1, min(int(n_splits), 64))
    if out is None:
        out = torch.empty((total_q, H, D), dtype=q.dtype, device=dev)
    lse = torch.empty((H, total_q), dtype=torch.float32, device=dev) if return_lse else None
    L = _hip.lib()
    ws = _hip.workspace(L.ls_sparse_attn_kvcache_workspace_size(total_q, G, n_splits), dev)
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    rc = L.ls_sparse_attn_kvcache(
        q.data_ptr(), q.stride(0), cu_seqlens_q.contiguous().data_ptr(), total_q,
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        cache_seqlens.contiguous().data_ptr(), B, H, G, D, _hip.dtype_code(q.dtype),
        topk_idx.data_ptr(), K, scale, 1 if causal else 0, n_splits, out.data_ptr(),
        _hip.ptr(lse), ws.data_ptr(), ws.numel(), _hip.stream_of(dev))
    _hip.check(rc, "ls_sparse_attn_kvcache")
    return (out, lse) if return_lse else out


def stage1_scores(q: torch.Tensor, kc: torch.Tensor, cu_seqlens_q: torch.Tensor,
                  cu_seqlens_kc: torch.Tensor, max_seqlen_k: int, *,
                  softmax_scale: float | None = None) -> torch.Tensor:
    """Decode-form stage-1 scores ``[G, total_q, max_seqlen_k]`` in ``q``'s dtype.

    ``out[g, t, j]`` is the sum over group ``g``'s query heads of
    ``softmax_j(scale * q[t, h] . kc[cu_seqlens_kc[b] + j, g])`` over the
    compressed keys of row ``t``'s sequence ``b`` (no causal limit), 0 past
    them and where the score is NaN (``infllmv2_attn_stage1`` with
    ``causal=False``, third_party/infllmv2/paper1.patch:2312-2361).  ``q
    [total_q, H, D]``; ``kc [total_kc, G, D]`` packed by ``cu_seqlens_kc``."""
    if q.ndim != 3 or kc.ndim != 3:
        raise ValueError("q must be [total_q, H, D] and kc [total_kc, G, D]")
    total_q, H, D = q.shape
    total_kc, G, Dk = kc.shape
    if Dk != D or H % G or q.dtype != kc.dtype:
        raise ValueError("q and kc must share head_dim and dtype, H divisible by G")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("stage-1 scores take bf16 or fp16 inputs")
    _hip.check_cu_seqlens(cu_seqlens_q, cu_seqlens_kc)
    dev = _hip.require_gpu(q, kc, cu_seqlens_q, cu_seqlens_kc)
    B = cu_seqlens_q.numel() - 1
    cu_host = [int(x) for x in cu_seqlens_kc.tolist()]
    max_kc = max((cu_host[b + 1] - cu_host[b] for b in range(B)), default=0)
    out_cols = int(max_seqlen_k)
    out = torch.zeros((G, total_q, out_cols), dtype=q.dtype, device=dev)
    if B == 0 or total_q == 0 or out_cols == 0:
        return out
    q = q if (q.stride(2) == 1 and q.stride(1) == D) else q.contiguous()
    kc = kc if (kc.stride(2) == 1 and kc.stride(1) == D) else kc.contiguous()
    L = _hip.lib()
    ws = _hip.workspace(L.ls_stage1_scores_workspace_size(total_q, G, max_kc), dev)
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    rc = L.ls_stage1_scores(
        q.data_ptr(), q.stride(0), cu_seqlens_q.contiguous().data_ptr(), total_q,
        kc.data_ptr() if total_kc else None, kc.stride(0), cu_seqlens_kc.contiguous().data_ptr(),
        B, max_kc, H, G, D, _hip.dtype_code(q.dtype), scale, out.data_ptr(), out_cols,
        ws.data_ptr(), ws.numel(), _hip.stream_of(dev))
    _hip.check(rc, "ls_stage1_scores")
    return out
