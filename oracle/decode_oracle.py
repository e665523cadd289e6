"""Decode restatements: the compressed-key cache update and stage-1 decode
selection (test infrastructure only; see the package docstring).

Pinning status:
- ``cache_windows_incremental``: pinned by equality with ``compress_k`` over the
  whole cache (a window is the same mean whether formed at prefill or when a
  decode token completes it) and by brute force on small caches.
- ``stage1_decode_scores``: the stage-1 kernel is not vendored in the
  reference (``third_party/infllmv2`` holds only a patch whose hunks show the
  causal rule and that the ``v`` operand is unused).  What is restated here is
  the operator's documented contract, softmax over the compressed keys per
  query head summed over the heads of a KV group, with ``causal=False`` as the
  decode call passes it (``minicpm.py:682-692``).  Pinned by the invariants
  that fix that contract (each row sums to the group size; one key gives the
  group size exactly) and by ``torch.softmax`` as the library routine.  Whether
  the kernel divides by the group size is not visible; the division is a power
  of two and cannot change a ranking, so the plans do not depend on it.
  The rounding of the per-key sums (kernel summation order) is unpinned.
- ``decode_select``: the pooling is ``page_maxpool_varlen`` (pinned with the
  NOSA oracle) and the selection tail is ``compressed_attention``'s
  (``minicpm.py:694-705``: ``topk``, ``sort``, ids past ``q_idx`` to -1);
  ``torch.topk`` leaves ties unspecified, here they go to the lower page.
"""
from __future__ import annotations

from typing import Sequence

import torch

from .leanselect_oracle import _as_list, _round, _stable_topk_desc
from .nosa_oracle import page_maxpool_varlen

__all__ = ["n_windows", "cache_windows_incremental", "stage1_decode_scores", "decode_select"]


def n_windows(length: int, kernel_size: int = 32, kernel_stride: int = 16) -> int:
    """Compressed windows of a ``length``-token sequence (``calc_chunks_with_stride``)."""
    return (length - kernel_size) // kernel_stride + 1 if length >= kernel_size else 0


def cache_windows_incremental(keys: torch.Tensor, step_lengths: Sequence[int],
                              kernel_size: int = 32, kernel_stride: int = 16) -> torch.Tensor:
    """Compressed windows of one sequence's keys ``[L, G, D]`` formed the way
    ``InfLLMv2CacheLayer`` forms them while tokens arrive in chunks of
    ``step_lengths`` (``minicpm.py:1308-1325, 2776-2823, 2888-2958``): the prefill
    chunk compresses its complete windows and keeps the tail from
    ``n_windows * stride``; each later chunk is appended to that tail, and
    whenever the tail holds ``kernel_size`` tokens its first ``kernel_size``
    rows are averaged and ``kernel_stride`` rows dropped.  Float64 means,
    rounded once to the key dtype."""
    kd = keys.detach().to(torch.float64)
    out = []
    first = int(step_lengths[0]) if len(step_lengths) else 0
    n0 = n_windows(first, kernel_size, kernel_stride)
    for w in range(n0):
        out.append(kd[w * kernel_stride: w * kernel_stride + kernel_size].mean(0))
    tail_start = n0 * kernel_stride
    pos = first
    for n in step_lengths[1:]:
        for _ in range(int(n)):
            pos += 1  # the tail now ends at pos
            if pos - tail_start >= kernel_size:
                out.append(kd[tail_start: tail_start + kernel_size].mean(0))
                tail_start += kernel_stride
    if not out:
        return keys.new_empty((0,) + tuple(keys.shape[1:]))
    return _round(torch.stack(out), keys.dtype)


def stage1_decode_scores(q: torch.Tensor, kc: torch.Tensor, cu_seqlens_q, cu_seqlens_kc, *,
                         softmax_scale: float | None = None,
                         rows: Sequence[int] | None = None) -> torch.Tensor:
    """``[G, R, max_kc]`` float64: for row ``t`` of sequence ``b`` and group ``g``,
    ``sum_{h in g} softmax_j(scale * q[t, h] . kc[j, g])`` over the sequence's
    compressed keys (no causal limit), 0 past them.  ``q [total_q, H, D]``,
    ``kc [total_kc, G, D]`` packed by ``cu_seqlens_kc``."""
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_kc)
    total_q, H, D = q.shape
    G = kc.shape[1]
    gs = H // G
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    max_kc = max((ck[b + 1] - ck[b] for b in range(len(ck) - 1)), default=0)
    row_list = list(range(total_q)) if rows is None else [int(r) for r in rows]
    out = torch.zeros((G, len(row_list), max_kc), dtype=torch.float64)
    qd = q.detach().to(torch.float64)
    kd = kc.detach().to(torch.float64)
    for i, t in enumerate(row_list):
        b = next(j for j in range(len(cq) - 1) if cq[j] <= t < cq[j + 1])
        k0, k1 = ck[b], ck[b + 1]
        if k1 <= k0:
            continue
        for g in range(G):
            s = scale * qd[t, g * gs:(g + 1) * gs] @ kd[k0:k1, g].T  # [gs, n]
            p = torch.exp(s - s.amax(dim=-1, keepdim=True))
            p = p / p.sum(dim=-1, keepdim=True)
            out[g, i, : k1 - k0] = p.sum(dim=0)
    return out


def decode_select(q: torch.Tensor, kc: torch.Tensor, cu_seqlens_q, cu_seqlens_kc, seqlens_k, *,
                  topk: int, init_blocks: int = 1, local_blocks: int = 32, block_size: int = 64,
                  kernel_stride: int = 16, softmax_scale: float | None = None,
                  return_scores: bool = False):
    """Stage-1 decode plans ``[G, total_q, min(topk, out_len)]`` int32.

    Row ``i`` of sequence ``b`` sits at position ``seqlens_k[b] - len_q(b) + i``
    (``seqlens_k`` counting the rows' own tokens; the reference's decode passes
    ``cache_lens = seq_lens_k - 1`` for one row, ``minicpm.py:2509-2512``).
    Scores are ``stage1_decode_scores`` rounded to the query dtype, then to
    bf16 (``minicpm.py:694-696``); pages by ``page_maxpool_varlen`` with
    ``cache_lens = seqlens_k - len_q``; the ``min(topk, out_len)`` best pages
    (ties to the lower page), sorted, ids past the row's page replaced by -1
    (``minicpm.py:697-704``).  With ``return_scores`` also the pooled page
    scores ``[G, total_q, out_len]`` (float64)."""
    cq = _as_list(cu_seqlens_q)
    ck = _as_list(cu_seqlens_kc)
    lens = _as_list(seqlens_k)
    batch = len(cq) - 1
    len_q = [cq[b + 1] - cq[b] for b in range(batch)]
    cache_lens = [lens[b] - len_q[b] for b in range(batch)]
    max_q = max(len_q, default=0)
    max_kc = max((ck[b + 1] - ck[b] for b in range(batch)), default=0)
    raw = stage1_decode_scores(q, kc, cq, ck, softmax_scale=softmax_scale)
    score = _round(_round(raw, q.dtype), torch.bfloat16) if q.dtype != torch.bfloat16 \
        else _round(raw, torch.bfloat16)
    pooled = page_maxpool_varlen(score, cq, ck, cache_lens, max_q, max_kc,
                                 local_blocks=local_blocks, init_blocks=init_blocks,
                                 block_size=block_size, stride=kernel_stride)
    pooled = pooled.to(torch.float64)
    out_len = pooled.shape[-1]
    k = min(int(topk), out_len)
    idx = _stable_topk_desc(pooled, k)
    idx = torch.sort(idx, dim=-1).values
    q_idx = torch.cat([(torch.arange(len_q[b]) + cache_lens[b]) // block_size
                       for b in range(batch)]) if batch else torch.zeros(0, dtype=torch.long)
    idx = idx.masked_fill(idx > q_idx[None, :, None], -1).to(torch.int32)
    # -1 entries sort last in the reference's list only because they replace the
    # largest ids; keep the kept ids first, then the padding.
    if return_scores:
        return idx, pooled
    return idx
