"""CIS mean pooling on the GPU (mirror of ``leanselect.ops.cis_pooling``).

``nosa_mean_pooling`` keeps the reference's signature
(leanselect/ops/cis_pooling.py:48-72) and runs ``ls_cis_mean_pool``.
"""
from __future__ import annotations

import torch

from .. import _hip

__all__ = ["nosa_mean_pooling"]


def nosa_mean_pooling(cis_score: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                      kernel_size: int = 32, stride: int = 16) -> torch.Tensor:
    """``cis_score [N, H] -> [H, N, max_seqlen // stride - 1]``.

    Entry ``[h, t, m]`` is the mean of the ``kernel_size`` CIS values of
    sequence ``b`` starting at token ``m * stride`` for every row ``t`` of ``b``
    when that window lies inside the sequence, else 0.  Summed in float32,
    rounded once to ``cis_score.dtype``.
    """
    if kernel_size != 32 or stride != 16:
        raise ValueError("nosa_mean_pooling supports kernel_size 32 and stride 16")
    if cis_score.ndim != 2:
        raise ValueError("cis_score must be [N, H]")
    dev = _hip.require_gpu(cis_score, cu_seqlens)
    if cu_seqlens.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32")
    N, H = cis_score.shape
    M = max(int(max_seqlen) // stride - 1, 0)
    out = torch.empty((H, N, M), dtype=cis_score.dtype, device=dev)
    if M == 0 or N == 0 or H == 0:
        return out
    if cis_score.stride(1) != 1:
        cis_score = cis_score.contiguous()
    rc = _hip.lib().ls_cis_mean_pool(
        cis_score.data_ptr(), cis_score.stride(0), N, H, cu_seqlens.contiguous().data_ptr(),
        cu_seqlens.numel() - 1, int(max_seqlen), kernel_size, stride,
        _hip.dtype_code(cis_score.dtype), out.data_ptr(), M, _hip.stream_of(dev))
    _hip.check(rc, "ls_cis_mean_pool")
    return out
