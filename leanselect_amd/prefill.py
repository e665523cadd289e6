"""One attention layer of LeanSelect sparse prefill on the GPU.

Follows the LeanSelect prefill branch of ``_sparse_attention_forward``
(leanselect/models/minicpm.py:2389-2772): compress the post-RoPE keys
(``compress_k``), select pages per KV group and token
(``_lightweight_compressed_attention``), then block-sparse attention over the
selected pages (``sparse_forward``).  Inputs are already unpadded/packed.
"""
from __future__ import annotations

import torch

from .ops.attention import sparse_attention
from .ops.compress import compress_k
from .ops.profiling import range_pop, range_push
from .ops.select import leanselect_prefill_topk_idx

__all__ = ["leanselect_sparse_prefill"]


def leanselect_sparse_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    selector,
    *,
    topk: int,
    local_blocks: int,
    init_blocks: int = 1,
    block_size: int = 64,
    kernel_size: int = 32,
    kernel_stride: int = 16,
    cu_seqlens_host: list[int] | None = None,
    return_topk_idx: bool = False,
):
    """``(out [total, H, D], topk_idx [G, total, take])`` for packed prefill sequences.

    ``topk`` is the total page budget (forced pages included), i.e. the
    reference's ``self.topk = topk + window_size // block_size``.
    """
    host = cu_seqlens_host if cu_seqlens_host is not None else cu_seqlens.tolist()
    max_len = max(host[i + 1] - host[i] for i in range(len(host) - 1))
    range_push("compress")
    kc, cu_c = compress_k(k, cu_seqlens, kernel_size=kernel_size, kernel_stride=kernel_stride,
                          cu_seqlens_host=host)
    range_pop()
    range_push("stage 1")
    ids = leanselect_prefill_topk_idx(
        q, kc, cu_seqlens, cu_c, selector, topk=topk, block_size=block_size,
        kernel_stride=kernel_stride, init_blocks=init_blocks, local_blocks=local_blocks,
        cu_seqlens_q_host=host)
    range_pop()
    range_push("stage 2")
    out = sparse_attention(q, k, v, cu_seqlens, cu_seqlens, max_len, max_len, ids,
                           causal=True, block_size=block_size)
    range_pop()
    return (out, ids) if return_topk_idx else out
