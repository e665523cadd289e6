"""Decode KV cache in HBM: the counterpart of the reference's ``InfLLMv2Cache``
(leanselect/models/minicpm.py:1188-1490) for the LeanSelect model.

All layers' keys (after RoPE), values and 32/16 compressed keys live in
preallocated device tensors ``[layers, batch, capacity, G, D]`` (capacity
rounded up to the 64-token page), so appending a token writes in place
instead of concatenating, and the compressed keys are extended by the windows
each step completes (``ls_kvcache_append``) instead of being kept as Python
lists.  A step of new tokens is written layer by layer between ``begin`` and
``end``; during the step ``seqlens_after`` holds the lengths including it.
"""
from __future__ import annotations

import torch

from .ops.decode import kvcache_append, n_windows

__all__ = ["LeanSelectKVCache"]


class LeanSelectKVCache:
    def __init__(self, num_layers: int, batch: int, capacity: int, num_kv_heads: int,
                 head_dim: int = 128, *, dtype: torch.dtype = torch.bfloat16, device="cuda",
                 kernel_size: int = 32, kernel_stride: int = 16):
        if num_layers < 1 or batch < 1 or capacity < 1:
            raise ValueError("num_layers, batch and capacity must be positive")
        cap = -(-int(capacity) // 64) * 64
        self.num_layers, self.batch, self.capacity = int(num_layers), int(batch), cap
        self.kernel_size, self.kernel_stride = int(kernel_size), int(kernel_stride)
        self.device = torch.device(device)
        shape = (num_layers, batch, cap, num_kv_heads, head_dim)
        self.k = torch.empty(shape, dtype=dtype, device=self.device)
        self.v = torch.empty(shape, dtype=dtype, device=self.device)
        cap_c = max(1, n_windows(cap, kernel_size, kernel_stride))
        self.kc = torch.empty((num_layers, batch, cap_c, num_kv_heads, head_dim), dtype=dtype,
                              device=self.device)
        self.lengths = [0] * batch  # tokens held before the open step
        self.seqlens = torch.zeros(batch, dtype=torch.int32, device=self.device)
        self._step = None

    # -- step protocol --------------------------------------------------------
    def begin(self, n_new: list[int]) -> None:
        """Open a step that appends ``n_new[b]`` tokens to sequence ``b``."""
        if self._step is not None:
            raise RuntimeError("a cache step is already open")
        if len(n_new) != self.batch or any(n < 0 for n in n_new):
            raise ValueError(f"n_new must hold {self.batch} non-negative counts")
        after = [l + n for l, n in zip(self.lengths, n_new)]
        if max(after) > self.capacity:
            raise ValueError(f"the step would exceed the cache capacity {self.capacity}")
        cu = [0]
        for n in n_new:
            cu.append(cu[-1] + int(n))
        self._step = dict(
            cu_host=cu, cu=torch.tensor(cu, dtype=torch.int32, device=self.device),
            after_host=after, after=torch.tensor(after, dtype=torch.int32, device=self.device))

    def update(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Write layer ``layer``'s packed new keys / values ``[sum n_new, G, D]``
        (and the compressed windows they complete) into the cache."""
        st = self._require_step()
        kvcache_append(self.k[layer], self.v[layer], self.seqlens, k_new, v_new, st["cu"],
                       kc_cache=self.kc[layer], kernel_size=self.kernel_size,
                       kernel_stride=self.kernel_stride, cache_seqlens_host=self.lengths,
                       cu_seqlens_new_host=st["cu_host"])

    def end(self) -> None:
        """Close the step: the appended tokens count from now on."""
        st = self._require_step()
        self.lengths = list(st["after_host"])
        self.seqlens = st["after"]
        self._step = None

    @property
    def seqlens_after(self) -> torch.Tensor:
        """int32 ``[batch]`` lengths including the open step."""
        return self._require_step()["after"]

    @property
    def lengths_after(self) -> list[int]:
        return list(self._require_step()["after_host"])

    def get_seq_length(self) -> int:
        """Tokens of the longest sequence (outside a step)."""
        return max(self.lengths)

    def _require_step(self):
        if self._step is None:
            raise RuntimeError("no cache step is open (call begin first)")
        return self._step
