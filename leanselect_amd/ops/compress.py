"""Compressed keys on the GPU (a1).

Mirrors ``CompressK`` / ``calc_chunks_with_stride``
(leanselect/models/minicpm.py:711-750, 1158-1185): the mean of every
``kernel_size``-token window at ``kernel_stride`` that lies inside one packed
sequence, computed by ``ls_compress_k_varlen``.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _hip

__all__ = ["CompressK", "compress_k", "compressed_lengths"]


def compressed_lengths(cu_seqlens_host: list[int], kernel_size: int, kernel_stride: int) -> list[int]:
    """Atoms per sequence: ``(len - kernel_size) // kernel_stride + 1`` or 0."""
    out = []
    for b in range(len(cu_seqlens_host) - 1):
        n = cu_seqlens_host[b + 1] - cu_seqlens_host[b]
        out.append((n - kernel_size) // kernel_stride + 1 if n >= kernel_size else 0)
    return out


def compress_k(
    k: torch.Tensor,
    cu_seqlens: torch.Tensor,
    *,
    kernel_size: int = 32,
    kernel_stride: int = 16,
    cu_seqlens_host: list[int] | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``k [total_k, G, D]`` -> ``(compressed_k [sum A, G, D], cu_seqlens_compressed int32)``."""
    if k.ndim != 3:
        raise ValueError(f"k must be [total_k, num_kv_heads, head_dim], got {tuple(k.shape)}")
    if kernel_size <= 0 or kernel_stride <= 0:
        raise ValueError("kernel_size and kernel_stride must be positive")
    dev = _hip.require_gpu(k, cu_seqlens)
    if cu_seqlens.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32")
    if k.stride(2) != 1 or k.stride(1) != k.shape[2]:
        k = k.contiguous()
    host = cu_seqlens_host if cu_seqlens_host is not None else cu_seqlens.tolist()
    batch = len(host) - 1
    total_atoms = sum(compressed_lengths(host, kernel_size, kernel_stride))
    G, D = k.shape[1], k.shape[2]
    out = torch.empty((total_atoms, G, D), dtype=k.dtype, device=dev)
    cu_out = torch.empty((batch + 1,), dtype=torch.int32, device=dev)
    cu = cu_seqlens.contiguous()
    rc = _hip.lib().ls_compress_k_varlen(
        k.data_ptr(), k.stride(0), cu.data_ptr(), batch, G, D, _hip.dtype_code(k.dtype),
        kernel_size, kernel_stride, out.data_ptr() if total_atoms else None, total_atoms,
        cu_out.data_ptr(), _hip.stream_of(dev))
    _hip.check(rc, "ls_compress_k_varlen")
    return out, cu_out


class CompressK(nn.Module):
    """Module form of :func:`compress_k` with the reference constructor."""

    def __init__(self, head_num_k: int, head_dim: int, kernel_size: int, kernel_stride: int = 16):
        super().__init__()
        self.kernel_size = kernel_size
        self.head_num_k = head_num_k
        self.head_dim = head_dim
        self.kernel_stride = kernel_stride

    def forward(self, k: torch.Tensor, cu_seqlens: torch.Tensor):
        return compress_k(k, cu_seqlens, kernel_size=self.kernel_size, kernel_stride=self.kernel_stride)
