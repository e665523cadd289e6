"""Drop-in for the native-op names the reference's model files import.

``leanselect/models/minicpm.py:78-98`` and ``nosa.py:1021-1039`` import these
names from ``infllm_v2``; ``load_model`` checks that they exist
(``leanselect/models/__init__.py:65-87``).  The LeanSelect prefill path uses
``infllmv2_attn_varlen_func(..., topk_idx=)``, NOSA's selection
``max_pooling_1d_varlen``, and decoding ``infllmv2_attn_with_kvcache(...,
topk_idx=)`` over the cache (the stage-1 decode selection itself is
``ops.decode_topk_idx``).  The stage-1 prefill selector, its KL-teacher form
and ``max_pooling_1d`` belong to the non-LeanSelect paths and raise
``NotImplementedError``.
"""
from __future__ import annotations

import torch

from .ops.attention import infllmv2_attn_varlen_func
from .ops.decode import kvcache_append, sparse_attention_kvcache
from .ops.nosa import max_pooling_1d_varlen

__all__ = [
    "infllmv2_attn_varlen_func",
    "infllmv2_attn_stage1",
    "infllmv2_attn_stage1_kl_teacher",
    "infllmv2_attn_with_kvcache",
    "max_pooling_1d",
    "max_pooling_1d_varlen",
]


def _not_provided(name: str):
    def fn(*args, **kwargs):
        raise NotImplementedError(f"{name} is outside the LeanSelect prefill hot path")

    fn.__name__ = name
    return fn


infllmv2_attn_stage1 = _not_provided("infllmv2_attn_stage1")
infllmv2_attn_stage1_kl_teacher = _not_provided("infllmv2_attn_stage1_kl_teacher")


def infllmv2_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None,
                               rotary_sin=None, cache_seqlens=None, cache_batch_idx=None,
                               cache_leftpad=None, block_table=None, softmax_scale=None,
                               causal=False, window_size=(-1, -1), softcap=0.0,
                               rotary_interleaved=True, alibi_slopes=None, num_splits=0,
                               return_softmax_lse=False, topk_idx=None):
    """Attention of ``q [B, Sq, H, D]`` over the cache ``k_cache / v_cache [B,
    capacity, G, D]`` holding ``cache_seqlens`` tokens per sequence, restricted to
    the pages of ``topk_idx [G, B * Sq, k]`` (every page when None).  With ``k /
    v [B, S_new, G, D]`` the new tokens are first written into the cache at
    ``cache_seqlens`` (in place) and attended too.  ``causal`` aligns row ``i``
    with key ``len - Sq + i``.  Returns ``out [B, Sq, H, D]`` (and
    ``softmax_lse [B, H, Sq]`` float32).  Follows the wrapper contract of
    ``third_party/infllmv2/paper1.patch:2511-2615``; rotary, paged
    (``block_table``), batch-index, left-pad, ALiBi, softcap and local-window
    options are not supported."""
    if any(x is not None for x in (rotary_cos, rotary_sin, cache_batch_idx, cache_leftpad,
                                   block_table, alibi_slopes)) or softcap != 0.0 \
            or tuple(window_size) != (-1, -1):
        raise NotImplementedError("infllmv2_attn_with_kvcache: rotary, paged, batch-index, "
                                  "left-pad, ALiBi, softcap and window options are not supported")
    if q.ndim != 4 or k_cache.ndim != 4:
        raise ValueError("q must be [B, Sq, H, D] and k_cache / v_cache [B, capacity, G, D]")
    B, Sq, H, D = q.shape
    G = k_cache.shape[2]
    dev = q.device
    if cache_seqlens is None:
        cache_seqlens = 0
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((B,), cache_seqlens, dtype=torch.int32, device=dev)
    if cache_seqlens.dtype != torch.int32:
        raise ValueError("cache_seqlens must be int32")
    lens = [int(x) for x in cache_seqlens.tolist()]
    if (k is None) != (v is None):
        raise ValueError("k and v must be given together")
    if k is not None:
        s_new = k.shape[1]
        cu_new = [b * s_new for b in range(B + 1)]
        kvcache_append(k_cache, v_cache, cache_seqlens, k.reshape(B * s_new, G, D),
                       v.reshape(B * s_new, G, D),
                       torch.tensor(cu_new, dtype=torch.int32, device=dev),
                       cache_seqlens_host=lens, cu_seqlens_new_host=cu_new)
        lens = [x + s_new for x in lens]
        cache_seqlens = torch.tensor(lens, dtype=torch.int32, device=dev)
    if topk_idx is None:  # every page of the longest sequence
        n_pages = max(1, -(-max(lens) // 64))
        topk_idx = torch.arange(n_pages, dtype=torch.int32, device=dev).expand(G, B * Sq, n_pages)
    cu_q = torch.arange(0, B * Sq + 1, Sq, dtype=torch.int32, device=dev)
    res = sparse_attention_kvcache(q.reshape(B * Sq, H, D), k_cache, v_cache, cache_seqlens,
                                   topk_idx, cu_q, causal=bool(causal),
                                   softmax_scale=softmax_scale,
                                   n_splits=num_splits if num_splits > 0 else None,
                                   return_lse=return_softmax_lse)
    if return_softmax_lse:
        out, lse = res
        return out.view(B, Sq, H, D), lse.view(H, B, Sq).permute(1, 0, 2).contiguous()
    return res.view(B, Sq, H, D)
max_pooling_1d = _not_provided("max_pooling_1d")
