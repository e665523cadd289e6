"""Compressed-key and page geometry with the reference interface.

Mirrors the eleven functions of ``leanselect/pages.py``.  The hot-path ones run
as gfx950 kernels on device tensors:

* ``compress_keys_mean``   (pages.py:84-101)   -> ``ls_compress_k_varlen``
* ``pool_atoms_to_pages``  (pages.py:146-187)  -> ``ls_pool_atoms_to_pages`` (``reduce="max"``)
* ``forced_page_mask``     (pages.py:222-240)  -> ``ls_forced_page_mask``

``group_size``, ``infllm_atom_count`` and ``serve_dynamic_k`` are host geometry.
The training/teacher helpers (``variable_k_topk_mask``, ``uniform_group_queries``,
``expand_kv_to_q_heads``, ``vanilla_atom_scores``, ``apply_atom_causal_mask``
and ``reduce="lse"`` pooling) are not on the prefill hot path; they are kept
for interface completeness as short torch compositions.
"""
from __future__ import annotations

import torch

from . import _hip

__all__ = [
    "serve_dynamic_k",
    "variable_k_topk_mask",
    "group_size",
    "uniform_group_queries",
    "infllm_atom_count",
    "compress_keys_mean",
    "expand_kv_to_q_heads",
    "vanilla_atom_scores",
    "pool_atoms_to_pages",
    "apply_atom_causal_mask",
    "forced_page_mask",
]


def serve_dynamic_k(topk: int, n_pages: int, forced_mask: torch.Tensor | None = None):
    """Free Top-K slots once forced pages take theirs (pages.py:7-23)."""
    cap = min(max(int(topk), 0), max(int(n_pages), 0))
    if forced_mask is None:
        return cap
    n_forced = forced_mask.to(dtype=torch.long).sum(dim=-1)
    return (cap - n_forced).clamp(min=0).clamp(max=int(n_pages) - n_forced)


def variable_k_topk_mask(scores: torch.Tensor, k) -> torch.Tensor:
    """True on each row's top-``k`` finite entries, ties to the lower index (pages.py:26-51)."""
    n = int(scores.shape[-1])
    if torch.is_tensor(k):
        kt = k.to(device=scores.device, dtype=torch.long)
        while kt.ndim < scores.ndim - 1:
            kt = kt.unsqueeze(0)
        kt = kt.expand(*scores.shape[:-1])
    else:
        kt = torch.full(scores.shape[:-1], int(k), device=scores.device, dtype=torch.long)
    order = torch.argsort(scores, dim=-1, descending=True, stable=True)
    rank = torch.empty_like(order).scatter_(
        -1, order, torch.arange(n, device=scores.device, dtype=order.dtype).expand_as(order))
    return (rank < kt.unsqueeze(-1)) & torch.isfinite(scores)


def group_size(num_q_heads: int, num_kv_heads: int) -> int:
    h, g = int(num_q_heads), int(num_kv_heads)
    if g <= 0 or h <= 0 or h % g:
        raise ValueError(f"H={h} must be a positive multiple of n_kv={g}")
    return h // g


def uniform_group_queries(q: torch.Tensor, num_kv_heads: int) -> torch.Tensor:
    """Mean query per GQA group ``(..., H, D) -> (..., G, D)`` (pages.py:62-71)."""
    g = int(num_kv_heads)
    gs = group_size(int(q.shape[-2]), g)
    return q.reshape(*q.shape[:-2], g, gs, int(q.shape[-1])).mean(dim=-2)


def infllm_atom_count(seq_len: int, kernel_size: int = 32, kernel_stride: int = 16) -> int:
    """Atoms of one sequence (pages.py:74-81); a short sequence still has one."""
    if min(seq_len, kernel_size, kernel_stride) <= 0:
        raise ValueError("sequence and compression geometry must be positive")
    return 1 if seq_len < kernel_size else (seq_len - kernel_size) // kernel_stride + 1


def compress_keys_mean(k: torch.Tensor, *, kernel_size: int = 32, kernel_stride: int = 16) -> torch.Tensor:
    """``[B, S, G, D] -> [B, C, G, D]`` window mean; S < kernel_size gives one whole-sequence atom."""
    if k.ndim != 4:
        raise ValueError(f"k must be [B, S, n_kv, D], got {tuple(k.shape)}")
    B, S, G, D = k.shape
    if min(S, kernel_size, kernel_stride) <= 0:
        raise ValueError("sequence and compression geometry must be positive")
    dev = _hip.require_gpu(k)
    ks, st = (S, S) if S < kernel_size else (kernel_size, kernel_stride)
    n = (S - ks) // st + 1
    kk = k.contiguous().reshape(B * S, G, D)
    cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32, device=dev)
    out = torch.empty((B * n, G, D), dtype=k.dtype, device=dev)
    cu_out = torch.empty((B + 1,), dtype=torch.int32, device=dev)
    rc = _hip.lib().ls_compress_k_varlen(
        kk.data_ptr(), G * D, cu.data_ptr(), B, G, D, _hip.dtype_code(k.dtype), ks, st,
        out.data_ptr() if out.numel() else None, B * n, cu_out.data_ptr(), _hip.stream_of(dev))
    _hip.check(rc, "ls_compress_k_varlen")
    return out.reshape(B, n, G, D)


def expand_kv_to_q_heads(k_atoms: torch.Tensor, num_q_heads: int) -> torch.Tensor:
    """``[B, C, G, D] -> [B, C, H, D]`` by repeating GQA groups (pages.py:104-112)."""
    g, h = int(k_atoms.shape[2]), int(num_q_heads)
    if g == h:
        return k_atoms
    if h % g:
        raise ValueError(f"H={h} is not a multiple of n_kv={g}")
    return k_atoms.repeat_interleave(h // g, dim=2)


def vanilla_atom_scores(q: torch.Tensor, k_4d: torch.Tensor) -> torch.Tensor:
    """Per-head teacher dots ``[B, Q, H, D] x [B, C, G, D] -> [B, Q, H, C]`` (pages.py:115-143)."""
    if q.ndim != 4 or k_4d.ndim != 4:
        raise ValueError("q must be [B,Q,H,D] and k [B,C,n_kv,D]")
    if q.shape[0] != k_4d.shape[0] or q.shape[-1] != k_4d.shape[-1]:
        raise ValueError("q/k batch or head_dim mismatch")
    B, Q, H, D = q.shape
    C, G = int(k_4d.shape[1]), int(k_4d.shape[2])
    gs = group_size(H, G)
    qb = q.view(B, Q, G, gs, D).permute(0, 2, 1, 3, 4).reshape(B * G, Q * gs, D).float()
    kb = k_4d.permute(0, 2, 1, 3).reshape(B * G, C, D).float().transpose(1, 2).contiguous()
    dots = torch.bmm(qb, kb)
    return dots.view(B, G, Q, gs, C).permute(0, 2, 1, 3, 4).reshape(B, Q, H, C).to(q.dtype)


def pool_atoms_to_pages(
    atom_scores: torch.Tensor,
    *,
    seq_len: int,
    block_size: int = 64,
    kernel_stride: int = 16,
    reduce: str = "max",
) -> torch.Tensor:
    """Overlapping-window page score ``[..., A] -> [..., ceil(seq_len / block_size)]``.

    Page ``p`` reads atoms ``[p*s - 1, p*s + s)`` with ``s = block_size //
    kernel_stride`` (pages.py:146-196); ``max`` runs on the GPU.
    """
    if min(seq_len, block_size, kernel_stride) <= 0:
        raise ValueError("page geometry must be positive")
    if atom_scores.ndim < 1 or atom_scores.shape[-1] == 0 or not atom_scores.is_floating_point():
        raise ValueError("atom_scores must be floating point with a nonempty atom dimension")
    if block_size % kernel_stride:
        raise ValueError(f"block_size={block_size} must be divisible by kernel_stride={kernel_stride}")
    if reduce not in ("max", "lse"):
        raise ValueError(f"reduce must be max or lse, got {reduce!r}")
    s = block_size // kernel_stride
    n_pages = (int(seq_len) + block_size - 1) // block_size
    n_atoms = int(atom_scores.shape[-1])
    if reduce == "lse":
        idx = torch.arange(n_pages, device=atom_scores.device)[:, None] * s - 1 + torch.arange(
            s + 1, device=atom_scores.device)
        valid = (idx >= 0) & (idx < n_atoms)
        g = atom_scores[..., idx.clamp(0, max(n_atoms - 1, 0))].masked_fill(~valid, float("-inf"))
        return torch.logsumexp(g.float(), dim=-1).to(atom_scores.dtype)
    dev = _hip.require_gpu(atom_scores)
    flat = atom_scores.reshape(-1, n_atoms)
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    out = torch.empty((flat.shape[0], n_pages), dtype=atom_scores.dtype, device=dev)
    rc = _hip.lib().ls_pool_atoms_to_pages(
        flat.data_ptr(), flat.shape[0], n_atoms, flat.stride(0),
        _hip.dtype_code(atom_scores.dtype), n_pages, s, out.data_ptr(), _hip.stream_of(dev))
    _hip.check(rc, "ls_pool_atoms_to_pages")
    return out.reshape(*atom_scores.shape[:-1], n_pages)


def apply_atom_causal_mask(
    atom_scores: torch.Tensor, query_abs_positions: torch.Tensor, *, kernel_stride: int = 16
) -> torch.Tensor:
    """Hide atoms starting after the query token (pages.py:199-219)."""
    n_atoms = int(atom_scores.shape[-1])
    start = torch.arange(n_atoms, device=atom_scores.device) * int(kernel_stride)
    pos = query_abs_positions.to(device=atom_scores.device)
    if pos.ndim == 1:
        pos = pos.view(1, -1).expand(atom_scores.shape[0], -1)
    while pos.ndim < atom_scores.ndim - 1:
        pos = pos.unsqueeze(-1)
    return atom_scores.masked_fill(~(start <= pos.unsqueeze(-1)), float("-inf"))


def forced_page_mask(
    query_abs_positions: torch.Tensor,
    *,
    num_pages: int,
    block_size: int = 64,
    init_blocks: int = 1,
    local_blocks: int = 32,
) -> torch.Tensor:
    """Sink and sliding local pages, ``[B, Q, num_pages]`` bool (pages.py:222-240)."""
    pos = query_abs_positions.long()
    if pos.ndim == 1:
        pos = pos.view(1, -1)
    dev = _hip.require_gpu(pos)
    pos = pos.contiguous()
    out = torch.empty((*pos.shape, int(num_pages)), dtype=torch.bool, device=dev)
    rc = _hip.lib().ls_forced_page_mask(
        pos.data_ptr(), pos.numel(), int(num_pages), int(block_size), int(init_blocks),
        int(local_blocks), out.data_ptr(), _hip.stream_of(dev))
    _hip.check(rc, "ls_forced_page_mask")
    return out
