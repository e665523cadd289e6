"""One attention layer of LeanSelect sparse prefill on the GPU.

Follows the LeanSelect prefill branch of ``_sparse_attention_forward``
(leanselect/models/minicpm.py:2389-2772): compress the post-RoPE keys
(``compress_k``), select pages per KV group and token
(``_lightweight_compressed_attention``), then block-sparse attention over the
selected pages (``sparse_forward``).  Inputs are already unpadded/packed.

``nosa_sparse_prefill`` is the LeanSelect branch of the NOSA layer's
``sparse_forward`` (leanselect/models/nosa.py:1980-2255): the same
compression, the two-stage qk/CIS selection (``compressed_attention``) and the
CIS-biased attention.
"""
from __future__ import annotations

import torch

from .ops.attention import sparse_attention
from .ops.compress import compress_k
from .ops.profiling import range_pop, range_push
from .ops.nosa import nosa_prefill_topk_idx, nosa_sparse_attention
from .ops.select import leanselect_prefill_topk_idx

__all__ = ["leanselect_sparse_prefill", "nosa_sparse_prefill"]


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
    compressed: tuple[torch.Tensor, torch.Tensor] | None = None,
    q_tilde: torch.Tensor | None = None,
):
    """``(out [total, H, D], topk_idx [G, total, take])`` for packed prefill sequences.

    ``topk`` is the total page budget (forced pages included), i.e. the
    reference's ``self.topk = topk + window_size // block_size``.
    ``compressed`` = ``(kc, cu_seqlens_compressed)`` when the producer of ``k``
    already formed the compressed keys (``minicpm.rope_k_compress``), and
    ``q_tilde`` the selector's projection of ``q`` when the producer of ``q``
    already formed it (``minicpm.rope_project_queries``).
    """
    host = cu_seqlens_host if cu_seqlens_host is not None else cu_seqlens.tolist()
    max_len = max(host[i + 1] - host[i] for i in range(len(host) - 1))
    range_push("compress")
    if compressed is not None:
        kc, cu_c = compressed
    else:
        kc, cu_c = compress_k(k, cu_seqlens, kernel_size=kernel_size,
                              kernel_stride=kernel_stride, cu_seqlens_host=host)
    range_pop()
    range_push("stage 1")
    ids = leanselect_prefill_topk_idx(
        q, kc, cu_seqlens, cu_c, selector, topk=topk, block_size=block_size,
        kernel_stride=kernel_stride, init_blocks=init_blocks, local_blocks=local_blocks,
        cu_seqlens_q_host=host, q_tilde=q_tilde)
    range_pop()
    range_push("stage 2")
    out = sparse_attention(q, k, v, cu_seqlens, cu_seqlens, max_len, max_len, ids,
                           causal=True, block_size=block_size)
    range_pop()
    return (out, ids) if return_topk_idx else out


def nosa_sparse_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cis: torch.Tensor,
    cu_seqlens: torch.Tensor,
    selector,
    *,
    topk: int = 96,
    init_blocks: int = 1,
    local_blocks: int = 16,
    select_blocks: int = 24,
    block_size: int = 64,
    kernel_size: int = 32,
    kernel_stride: int = 16,
    cu_seqlens_host: list[int] | None = None,
    return_topk_idx: bool = False,
    pool_clip: str = "sequence",
):
    """``(out [total, H, D], topk_idx [G, total, take])`` of a NOSA layer.

    ``cis [total, G]`` are the per-token eviction scores.  The selection scores
    the post-RoPE queries, as the LeanSelect branch does (nosa.py:2011-2019).
    ``pool_clip`` is the page max-pool's column range (``"sequence"`` or
    ``"row"``, as in ``nosa_prefill_topk_idx``).
    """
    host = cu_seqlens_host if cu_seqlens_host is not None else cu_seqlens.tolist()
    max_len = max(host[i + 1] - host[i] for i in range(len(host) - 1))
    range_push("compress")
    kc, cu_c = compress_k(k, cu_seqlens, kernel_size=kernel_size, kernel_stride=kernel_stride,
                          cu_seqlens_host=host)
    range_pop()
    range_push("stage 1")
    ids = nosa_prefill_topk_idx(
        q, kc, cis, cu_seqlens, cu_c, cu_seqlens, selector,
        topk=topk, init_blocks=init_blocks, local_blocks=local_blocks,
        select_blocks=select_blocks, block_size=block_size, kernel_stride=kernel_stride,
        max_seqlen_q=max_len, cu_seqlens_q_host=host, pool_clip=pool_clip)
    range_pop()
    range_push("stage 2")
    out = nosa_sparse_attention(q, k, v, cis, cu_seqlens, cu_seqlens, max_len, max_len, ids,
                                block_size=block_size)
    range_pop()
    return (out, ids) if return_topk_idx else out
