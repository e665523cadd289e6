"""Drop-in for the native-op names the reference's model files import.

``leanselect/models/minicpm.py:78-98`` and ``nosa.py:1021-1039`` import these
names from ``infllm_v2``; ``load_model`` checks that they exist
(``leanselect/models/__init__.py:65-87``).  The LeanSelect prefill path uses
``infllmv2_attn_varlen_func(..., topk_idx=)``, NOSA's selection
``max_pooling_1d_varlen``, and decoding ``infllmv2_attn_stage1(...,
causal=False)`` (the stage-1 scores that ``compressed_attention`` pools and
ranks when decoding, minicpm.py:673-705) and ``infllmv2_attn_with_kvcache(...,
topk_idx=)`` over the cache (``ops.decode_topk_idx`` runs the whole stage-1
decode selection in one call).  The causal (prefill) stage-1 selector, its
KL-teacher form and ``max_pooling_1d`` belong to the non-LeanSelect paths and
raise ``NotImplementedError``.
"""
from __future__ import annotations

import torch

from .ops.attention import infllmv2_attn_varlen_func
from .ops.decode import kvcache_append, sparse_attention_kvcache, stage1_scores
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


def infllmv2_attn_stage1(q, k, v, cu_seqlens_q, cu_seqlens_k, cu_seqlens_v=None,
                         max_seqlen_q=None, max_seqlen_k=None, dropout_p=0.0,
                         softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                         alibi_slopes=None, deterministic=False, return_attn_probs=False,
                         block_table=None):
    """Stage-1 scores ``[nheads_k, total_q, max_seqlen_k]`` in ``q``'s dtype:
    for each query row and KV group, the group's per-head softmax over the
    row's sequence of compressed keys ``k`` (packed by ``cu_seqlens_k``),
    summed over the group's heads; 0 past the sequence's keys and where NaN
    (third_party/infllmv2/paper1.patch:2312-2361).  The decode form only
    (``causal=False``, as ``compressed_attention`` calls it with ``cache_lens``,
    leanselect/models/minicpm.py:617-683); ``v`` / ``cu_seqlens_v`` are accepted
    and unused, as the scores do not read values."""
    del v, cu_seqlens_v, max_seqlen_q, deterministic, return_attn_probs
    if causal:
        raise NotImplementedError("infllmv2_attn_stage1: only the decode form (causal=False) is "
                                  "provided; the causal prefill selector is not on the LeanSelect path")
    if dropout_p or tuple(window_size) != (-1, -1) or softcap or alibi_slopes is not None \
            or block_table is not None:
        raise NotImplementedError("infllmv2_attn_stage1: dropout / window / softcap / alibi / "
                                  "block_table are not supported")
    if max_seqlen_k is None:
        cu = [int(x) for x in cu_seqlens_k.tolist()]
        max_seqlen_k = max((cu[i + 1] - cu[i] for i in range(len(cu) - 1)), default=0)
    return stage1_scores(q, k, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_k),
                         softmax_scale=softmax_scale)


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
    cu_q = torch.arange(0, B * Sq + 1, Sq, dtype=torch.int32, device=dev)
    qr = q.reshape(B * Sq, H, D)
    splits = num_splits if num_splits > 0 else None
    if topk_idx is None:  # every page of the longest sequence
        out, lse = _dense_kvcache(qr, k_cache, v_cache, cache_seqlens, cu_q, max(lens), G,
                                  bool(causal), softmax_scale, splits)
    else:
        res = sparse_attention_kvcache(qr, k_cache, v_cache, cache_seqlens, topk_idx, cu_q,
                                       causal=bool(causal), softmax_scale=softmax_scale,
                                       n_splits=splits, return_lse=return_softmax_lse)
        out, lse = res if return_softmax_lse else (res, None)
    if return_softmax_lse:
        return out.view(B, Sq, H, D), lse.view(H, B, Sq).permute(1, 0, 2).contiguous()
    return out.view(B, Sq, H, D)


_KV_MAX_IDS = 256  # ids per row of one ls_sparse_attn_kvcache call


def _dense_kvcache(q, k_cache, v_cache, cache_seqlens, cu_q, max_len, G, causal, softmax_scale,
                   n_splits):
    """Attention over every cached page (``blockmask=None`` in the reference).

    A row of one kvcache call holds at most 256 page ids, so a cache of more
    pages is attended in groups of 256 pages whose partial results are merged
    by their log-sum-exp: ``out = sum_i w_i out_i / sum_i w_i`` with ``w_i =
    exp(lse_i - max lse)``; a group with no visible key (``lse = +inf``, ``out
    = 0``) gets weight 0.  Each partial output is rounded to the activation
    dtype before the merge, which is done in float32."""
    n_pages = max(1, -(-max_len // 64))
    total_q, H, _ = q.shape
    dev = q.device
    parts = []
    for p0 in range(0, n_pages, _KV_MAX_IDS):
        n = min(_KV_MAX_IDS, n_pages - p0)
        ids = torch.arange(p0, p0 + n, dtype=torch.int32, device=dev).expand(G, total_q, n)
        parts.append(sparse_attention_kvcache(q, k_cache, v_cache, cache_seqlens, ids, cu_q,
                                              causal=causal, softmax_scale=softmax_scale,
                                              n_splits=n_splits, return_lse=True))
    if len(parts) == 1:
        return parts[0]
    lses = torch.stack([lse for _, lse in parts])               # [P, H, total_q]
    lses = torch.where(torch.isinf(lses) & (lses > 0), torch.full_like(lses, float("-inf")), lses)
    m = lses.amax(dim=0)
    m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    w = torch.exp(lses - m_safe)                                  # [P, H, total_q]
    wsum = w.sum(dim=0)
    acc = torch.zeros(total_q, H, q.shape[2], dtype=torch.float32, device=dev)
    for (o, _), wi in zip(parts, w):
        acc += o.float() * wi.t().unsqueeze(-1)
    has = wsum > 0
    inv = torch.where(has, 1.0 / torch.where(has, wsum, torch.ones_like(wsum)), torch.zeros_like(wsum))
    out = (acc * inv.t().unsqueeze(-1)).to(q.dtype)
    lse = torch.where(has, m_safe + torch.log(torch.where(has, wsum, torch.ones_like(wsum))),
                      torch.full_like(wsum, float("inf")))
    return out, lse


max_pooling_1d = _not_provided("max_pooling_1d")
