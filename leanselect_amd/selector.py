"""LeanSelect router with the reference interface, computed by the HIP library.

Mirrors ``leanselect/selector.py``: the same constants, supervision-window
helpers, ``LeanSelectSelector`` constructor, parameters (float32 masters
``head_mix [H, R]``, ``kv_head_mix [G, R]``, ``q_proj [R, D, F]``,
``k_proj [R, D, F]``, each tagged ``_is_indexer``), initialisation recipe and
methods.  ``fused_weights``, ``project_queries``, ``project_atom_keys`` and
``score_pages`` run as gfx950 kernels on device tensors; they are forward-only
(selector training is not part of this package).
"""
from __future__ import annotations

import torch
from torch import nn

from . import _hip

LEANSELECT_INITIALIZATION = "gqa_mean_raw_dot_atom_max_orthogonal_frame_v2"
LEANSELECT_SUPERVISION_MAX_WINDOWS = 64
LEANSELECT_SUPERVISION_WINDOW_POLICY = "up_to_64_disjoint_windows_uniform_over_nontrivial_history"
LEANSELECT_CANONICAL_TENSORS = ("head_mix", "kv_head_mix", "q_proj", "k_proj")

__all__ = [
    "LEANSELECT_INITIALIZATION",
    "LEANSELECT_SUPERVISION_MAX_WINDOWS",
    "LEANSELECT_SUPERVISION_WINDOW_POLICY",
    "LEANSELECT_CANONICAL_TENSORS",
    "leanselect_supervision_windows",
    "leanselect_informative_history_start",
    "LeanSelectSelector",
]


def leanselect_supervision_windows(
    sequence_length: int,
    supervision_rows: int,
    *,
    max_windows: int = LEANSELECT_SUPERVISION_MAX_WINDOWS,
    minimum_start: int = 0,
) -> tuple[tuple[int, int], ...]:
    """Disjoint contiguous row windows ending at ``sequence_length``.

    Same contract as leanselect/selector.py:13-54: ``min(supervision_rows,
    sequence_length - minimum_start)`` rows split into at most ``max_windows``
    windows whose widths differ by at most one (wider windows first), with the
    spare history distributed as gaps (larger gaps last), the first window at
    ``minimum_start`` and the last one ending at ``sequence_length``.
    """
    n, rows, cap, lo = (int(sequence_length), int(supervision_rows), int(max_windows),
                        int(minimum_start))
    if n <= 0 or rows <= 0 or cap <= 0:
        raise ValueError("LeanSelect supervision geometry must be positive")
    if not 0 <= lo < n:
        raise ValueError("LeanSelect minimum_start must be inside the sequence")
    history = n - lo
    used = min(history, rows)
    if used == history:
        return ((lo, n),)
    count = min(cap, used)
    q, rem = divmod(used, count)
    sizes = [q + 1 if i < rem else q for i in range(count)]
    if count == 1:
        return ((n - sizes[0], n),)
    spare = history - used
    gq, grem = divmod(spare, count - 1)
    # The last `grem` gaps take the extra row.
    gaps = [gq + 1 if i >= count - 1 - grem else gq for i in range(count - 1)]
    out = []
    pos = lo
    for i, size in enumerate(sizes):
        out.append((pos, pos + size))
        pos += size + (gaps[i] if i < count - 1 else 0)
    if out[-1][1] != n:
        raise RuntimeError("LeanSelect supervision windows do not span the sequence")
    return tuple(out)


def leanselect_informative_history_start(*, total_topk_blocks: int, block_size: int) -> int:
    """First supervised row: twice the Top-K budget in tokens (selector.py:57-66)."""
    total, bs = int(total_topk_blocks), int(block_size)
    if total <= 0 or bs <= 0:
        raise ValueError("LeanSelect Top-K and block size must be positive")
    return 2 * total * bs


class LeanSelectSelector(nn.Module):
    """Low-rank per-GQA-group router (one page plan per KV group and token)."""

    def __init__(
        self,
        *,
        num_heads: int,
        num_kv_heads: int,
        head_dim: int,
        router_heads: int = 4,
        router_dim: int = 32,
    ) -> None:
        super().__init__()
        dims = dict(num_heads=int(num_heads), num_kv_heads=int(num_kv_heads),
                    head_dim=int(head_dim), router_heads=int(router_heads),
                    router_dim=int(router_dim))
        if min(dims.values()) <= 0:
            raise ValueError("all LeanSelect dimensions must be positive")
        if dims["router_heads"] > dims["num_heads"]:
            raise ValueError("router_heads cannot exceed num_heads")
        if dims["num_heads"] % dims["num_kv_heads"]:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        for k, v in dims.items():
            setattr(self, k, v)
        R, D, F = self.router_heads, self.head_dim, self.router_dim
        self.head_mix = nn.Parameter(torch.empty(self.num_heads, R))
        self.kv_head_mix = nn.Parameter(torch.empty(self.num_kv_heads, R))
        self.q_proj = nn.Parameter(torch.empty(R, D, F))
        self.k_proj = nn.Parameter(torch.empty(R, D, F))
        for p in self.parameters():
            p._is_indexer = True
        self.reset_parameters()

    # -- parameters --------------------------------------------------------
    def reset_parameters(self) -> None:
        """Group-mean mixing and a shared orthonormal frame scaled by D^-1/4.

        Same recipe as leanselect/selector.py:112-137, so at initialisation
        q~ . k~ equals the group-mean query dot the key over sqrt(D) whenever
        R * F == D.
        """
        with torch.no_grad():
            gs = self.num_heads // self.num_kv_heads
            self.head_mix.fill_(1.0 / gs)
            self.kv_head_mix.fill_(1.0)
            width = self.router_heads * self.router_dim
            if width <= self.head_dim:
                frame = torch.linalg.qr(
                    torch.randn(self.head_dim, width, dtype=torch.float32), mode="reduced").Q
            else:
                frame = torch.linalg.qr(
                    torch.randn(width, self.head_dim, dtype=torch.float32), mode="reduced").Q.T
            frame = frame * self.head_dim ** -0.25
            proj = frame.reshape(self.head_dim, self.router_heads, self.router_dim).permute(1, 0, 2)
            self.q_proj.copy_(proj)
            self.k_proj.copy_(proj)

    def canonical_state(self) -> dict[str, torch.Tensor]:
        """Canonical float32 masters (the fused weights are derived state)."""
        return {name: getattr(self, name) for name in LEANSELECT_CANONICAL_TENSORS}

    def _masters(self) -> list[torch.Tensor]:
        if torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()):
            raise RuntimeError(
                "LeanSelectSelector kernels are forward-only; call under torch.no_grad() "
                "or with requires_grad_(False)")
        return [getattr(self, n).detach().float().contiguous() for n in LEANSELECT_CANONICAL_TENSORS]

    def _workspace(self, dev, total_q: int, n_atoms: int, dt: int) -> torch.Tensor:
        n = _hip.lib().ls_select_workspace_size(
            total_q, n_atoms, 0, self.num_heads, self.num_kv_heads, self.head_dim,
            self.router_heads, self.router_dim, 0, dt)
        return _hip.workspace(n, dev)

    # -- deploy-time computation -------------------------------------------
    def fused_weights(self, *, dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """``(q_fused [H, D, R*F], kv_fused [G, D, R*F])`` in ``dtype`` (default float32)."""
        hm, khm, qp, kp = self._masters()
        dev = _hip.require_gpu(hm)
        dtype = torch.float32 if dtype is None else dtype
        F = self.router_heads * self.router_dim
        qf = torch.empty((self.num_heads, self.head_dim, F), dtype=dtype, device=dev)
        kf = torch.empty((self.num_kv_heads, self.head_dim, F), dtype=dtype, device=dev)
        rc = _hip.lib().ls_fused_weights(
            hm.data_ptr(), khm.data_ptr(), qp.data_ptr(), kp.data_ptr(), self.num_heads,
            self.num_kv_heads, self.head_dim, self.router_heads, self.router_dim,
            _hip.dtype_code(dtype), qf.data_ptr(), kf.data_ptr(), _hip.stream_of(dev))
        _hip.check(rc, "ls_fused_weights")
        return qf, kf

    def project_queries(self, query: torch.Tensor) -> torch.Tensor:
        """``query [N, H, D] -> [G, N, R*F]`` in ``query.dtype``."""
        if query.ndim != 3 or tuple(query.shape[1:]) != (self.num_heads, self.head_dim):
            raise ValueError("query must have shape [N, num_heads, head_dim]")
        hm, _, qp, _ = self._masters()
        dev = _hip.require_gpu(query, hm)
        query = query.detach()
        if query.stride(2) != 1 or query.stride(1) != self.head_dim:
            query = query.contiguous()
        dt = _hip.dtype_code(query.dtype)
        F = self.router_heads * self.router_dim
        out = torch.empty((self.num_kv_heads, query.shape[0], F), dtype=query.dtype, device=dev)
        ws = self._workspace(dev, 0, 0, dt)
        rc = _hip.lib().ls_project_queries(
            query.data_ptr(), query.stride(0), query.shape[0], self.num_heads, self.num_kv_heads,
            self.head_dim, hm.data_ptr(), qp.data_ptr(), self.router_heads, self.router_dim, dt,
            out.data_ptr(), ws.data_ptr(), ws.numel(), _hip.stream_of(dev))
        _hip.check(rc, "ls_project_queries")
        return out

    def project_atom_keys(self, compressed_keys: torch.Tensor) -> torch.Tensor:
        """``compressed_keys [A, G, D] -> [G, A, R*F]`` in the keys' dtype."""
        if compressed_keys.ndim != 3 or tuple(compressed_keys.shape[1:]) != (
                self.num_kv_heads, self.head_dim):
            raise ValueError("compressed_keys must have shape [A, num_kv_heads, head_dim]")
        _, khm, _, kp = self._masters()
        dev = _hip.require_gpu(compressed_keys, khm)
        kc = compressed_keys.detach()
        if kc.stride(2) != 1 or kc.stride(1) != self.head_dim:
            kc = kc.contiguous()
        dt = _hip.dtype_code(kc.dtype)
        F = self.router_heads * self.router_dim
        out = torch.empty((self.num_kv_heads, kc.shape[0], F), dtype=kc.dtype, device=dev)
        ws = self._workspace(dev, 0, 0, dt)
        rc = _hip.lib().ls_project_atom_keys(
            kc.data_ptr(), kc.stride(0), kc.shape[0], self.num_kv_heads, self.head_dim,
            khm.data_ptr(), kp.data_ptr(), self.router_heads, self.router_dim, dt,
            out.data_ptr(), ws.data_ptr(), ws.numel(), _hip.stream_of(dev))
        _hip.check(rc, "ls_project_atom_keys")
        return out

    def score_pages(
        self,
        query: torch.Tensor,
        compressed_keys: torch.Tensor,
        *,
        seq_len: int,
        block_size: int,
        kernel_stride: int,
    ) -> torch.Tensor:
        """Page scores ``[G, N, ceil(seq_len / block_size)]`` (selector.py:192-214)."""
        if query.ndim != 3 or tuple(query.shape[1:]) != (self.num_heads, self.head_dim):
            raise ValueError("query must have shape [N, num_heads, head_dim]")
        if compressed_keys.ndim != 3 or tuple(compressed_keys.shape[1:]) != (
                self.num_kv_heads, self.head_dim):
            raise ValueError("compressed_keys must have shape [A, num_kv_heads, head_dim]")
        seq_len, block_size, kernel_stride = int(seq_len), int(block_size), int(kernel_stride)
        if min(seq_len, block_size, kernel_stride) <= 0:
            raise ValueError("page geometry must be positive")
        if block_size % kernel_stride:
            raise ValueError(
                f"block_size={block_size} must be divisible by kernel_stride={kernel_stride}")
        if compressed_keys.shape[0] == 0:
            raise ValueError("atom_scores must be floating point with a nonempty atom dimension")
        if query.dtype != compressed_keys.dtype:
            raise ValueError("query and compressed_keys must share a dtype")
        hm, khm, qp, kp = self._masters()
        dev = _hip.require_gpu(query, compressed_keys, hm)
        q = query.detach()
        kc = compressed_keys.detach()
        if q.stride(2) != 1 or q.stride(1) != self.head_dim:
            q = q.contiguous()
        if kc.stride(2) != 1 or kc.stride(1) != self.head_dim:
            kc = kc.contiguous()
        dt = _hip.dtype_code(q.dtype)
        n_pages = (seq_len + block_size - 1) // block_size
        out = torch.empty((self.num_kv_heads, q.shape[0], n_pages), dtype=q.dtype, device=dev)
        ws = self._workspace(dev, q.shape[0], kc.shape[0], dt)
        rc = _hip.lib().ls_score_pages(
            q.data_ptr(), q.stride(0), q.shape[0], kc.data_ptr(), kc.stride(0), kc.shape[0],
            self.num_heads, self.num_kv_heads, self.head_dim, hm.data_ptr(), khm.data_ptr(),
            qp.data_ptr(), kp.data_ptr(), self.router_heads, self.router_dim, dt, seq_len,
            block_size, kernel_stride, out.data_ptr(), ws.data_ptr(), ws.numel(),
            _hip.stream_of(dev))
        _hip.check(rc, "ls_score_pages")
        return out
