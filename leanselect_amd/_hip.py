"""ctypes binding of ``libleanselect_hip.so`` (the C ABI in include/leanselect_hip.h).

The library is built in-tree by ``leanselect_amd.build``.  Loading fails loudly
when it is missing: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
from collections import deque
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libleanselect_hip.so")

LS_F32, LS_BF16, LS_F16 = 0, 1, 2
LS_OK, LS_ERR_INVALID, LS_ERR_UNSUPPORTED, LS_ERR_WORKSPACE, LS_ERR_HIP = range(5)
LS_ATTN_RING_TIMEOUT = 1
LS_POOL_CLIP_SEQUENCE, LS_POOL_CLIP_ROW = 0, 1
POOL_CLIPS = {"sequence": LS_POOL_CLIP_SEQUENCE, "row": LS_POOL_CLIP_ROW}


def pool_clip_code(clip: str) -> int:
    try:
        return POOL_CLIPS[clip]
    except KeyError:
        raise ValueError(f"unknown pool clip {clip!r}; expected 'sequence' or 'row'") from None

_i32, _i64, _f32, _sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
_p = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/leanselect_hip.h.
SIGNATURES = {
    "ls_version": (_i32, []),
    "ls_last_error": (ctypes.c_char_p, []),
    "ls_compress_k_varlen": (
        _i32, [_p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p, _p]),
    "ls_fused_weights": (
        _i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "ls_select_workspace_size": (
        _sz, [_i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "ls_project_queries": (
        _i32, [_p, _i64, _i64, _i32, _i32, _i32, _p, _p, _i32, _i32, _i32, _p, _p, _sz, _p]),
    "ls_rope_project_queries": (
        _i32, [_p, _i64, _p, _i64, _i32, _i32, _i32, _p, _p, _i64, _p, _p, _i32, _i32, _i32, _p,
               _p, _sz, _p]),
    "ls_project_atom_keys": (
        _i32, [_p, _i64, _i64, _i32, _i32, _p, _p, _i32, _i32, _i32, _p, _p, _sz, _p]),
    "ls_score_pages": (
        _i32, [_p, _i64, _i64, _p, _i64, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _i32, _i32,
               _i32, _i64, _i32, _i32, _p, _p, _sz, _p]),
    "ls_pool_atoms_to_pages": (_i32, [_p, _i64, _i64, _i64, _i32, _i64, _i32, _p, _p]),
    "ls_forced_page_mask": (_i32, [_p, _i64, _i64, _i32, _i32, _i32, _p, _p]),
    "ls_select_prefill": (
        _i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p,
               _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i32, _p, _sz, _p]),
    "ls_select_prefill_qt": (
        _i32, [_p, _i64, _p, _i64, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _i32, _i32,
               _i32, _i32, _i32, _i32, _i32, _i32, _p, _i32, _p, _sz, _p]),
    "ls_sparse_attn_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "ls_attn_set_spin_limit": (_i32, [_i32]),
    "ls_sparse_attn_varlen_noalloc": (
        _i32, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _i32, _i64, _i64, _i32, _i32, _i32, _i32,
               _i32, _i32, _p, _i32, _i32, _f32, _i32, _p, _p, _p, _p]),
    "ls_sparse_attn_varlen": (
        _i32, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _i32, _i64, _i64, _i32, _i32, _i32, _i32,
               _i32, _i32, _p, _i32, _i32, _f32, _i32, _p, _p, _p, _sz, _p]),
    "ls_cis_mean_pool": (
        _i32, [_p, _i64, _i64, _i32, _p, _i32, _i32, _i32, _i32, _i32, _p, _i32, _p]),
    "ls_page_maxpool_varlen": (
        _i32, [_p, _p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32,
               _p, _p]),
    "ls_nosa_select_workspace_size": (
        _sz, [_i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "ls_nosa_select_prefill": (
        _i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _p, _i32, _i32, _i32,
               _i32, _i32, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
               _i32, _p, _i32, _p, _sz, _p]),
    "ls_nosa_attn_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "ls_nosa_attn_varlen": (
        _i32, [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i32, _p, _p, _i32, _i64, _i64, _i32,
               _i32, _i32, _i32, _i32, _i32, _p, _i32, _i32, _f32, _p, _p, _p, _sz, _p]),
    "ls_rmsnorm": (_i32, [_p, _i64, _p, _i64, _i32, _f32, _i32, _p, _i64, _p]),
    "ls_add_rmsnorm": (
        _i32, [_p, _i64, _p, _i64, _f32, _p, _i64, _i32, _f32, _i32, _p, _i64, _p]),
    "ls_rope_inplace": (
        _i32, [_p, _i64, _p, _i64, _i32, _i32, _i64, _i32, _p, _p, _i64, _i32, _p]),
    "ls_rope_k_compress_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "ls_rope_k_compress": (
        _i32, [_p, _i64, _p, _p, _i32, _i64, _i32, _i64, _i32, _p, _p, _i64, _i32, _p, _i64, _p,
               _p, _sz, _p]),
    "ls_silu_mul": (_i32, [_p, _i64, _i64, _i32, _i32, _p, _i64, _p]),
    "ls_embed_scale": (_i32, [_p, _i64, _p, _i64, _i32, _f32, _i32, _p, _p]),
    "ls_kvcache_append": (
        _i32, [_p, _p, _i64, _i64, _p, _p, _p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _p, _i64,
               _i64, _i64, _i32, _i32, _p, _p]),
    "ls_decode_select_workspace_size": (_sz, [_i64, _i32, _i32, _i64, _i64]),
    "ls_decode_select": (
        _i32, [_p, _i64, _p, _i64, _p, _i64, _i64, _p, _i32, _i64, _i32, _i32, _i32, _i32, _f32,
               _i32, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _p, _p, _sz, _p]),
    "ls_stage1_scores_workspace_size": (_sz, [_i64, _i32, _i64]),
    "ls_stage1_scores": (
        _i32, [_p, _i64, _p, _i64, _p, _i64, _p, _i32, _i64, _i32, _i32, _i32, _i32, _f32, _p,
               _i64, _p, _sz, _p]),
    "ls_sparse_attn_kvcache_workspace_size": (_sz, [_i64, _i32, _i32]),
    "ls_sparse_attn_kvcache": (
        _i32, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _p, _i32, _i32, _i32, _i32, _i32, _p,
               _i32, _f32, _i32, _i32, _p, _p, _p, _sz, _p]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises RuntimeError when it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m leanselect_amd.build` "
                "(the LeanSelect hot path has no non-HIP implementation)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return {torch.float32: LS_F32, torch.bfloat16: LS_BF16, torch.float16: LS_F16}[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16")


def check(rc: int, name: str) -> None:
    if rc != LS_OK:
        msg = lib().ls_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must share one GPU device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"leanselect_amd runs on the GPU; got a tensor on {t.device} "
                "(move inputs to a ROCm device)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor argument")
    return dev


def check_cu_seqlens(cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor) -> None:
    """Both prefix-offset arrays must be 1-D int32 of the same length (the kernels
    read them as int32 ``[batch + 1]``)."""
    for name, t in (("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k)):
        if t.dtype != torch.int32 or t.ndim != 1 or t.numel() < 1:
            raise ValueError(f"{name} must be a 1-D int32 tensor of batch + 1 offsets, "
                             f"got {t.dtype} {tuple(t.shape)}")
    if cu_seqlens_q.numel() != cu_seqlens_k.numel():
        raise ValueError(f"cu_seqlens_q and cu_seqlens_k differ in length "
                         f"({cu_seqlens_q.numel()} != {cu_seqlens_k.numel()})")


def check_out(out: torch.Tensor, shape: tuple, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A caller-given output must be contiguous with exactly the output's shape,
    dtype and device (the kernels write it densely)."""
    if (tuple(out.shape) != tuple(shape) or out.dtype != dtype or out.device != device
            or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous {tuple(shape)} {dtype} tensor on {device}, "
                         f"got {tuple(out.shape)} {out.dtype} on {out.device}"
                         f"{'' if out.is_contiguous() else ' (not contiguous)'}")
    return out


class _StatusQueue:
    """Attention status words read without stalling the host.

    Each eager attention call queues a non-blocking copy of its workspace's
    status word into pinned host memory, followed by an event; the word is
    inspected once that event has completed -- at a later call's poll, or at
    ``attn_status_sync``.  So no call waits for its own kernels, and a wait that
    expired is reported by the first poll that finds the copy done."""

    MAX_PENDING = 64

    def __init__(self) -> None:
        self.pending: deque = deque()

    def push(self, ws: torch.Tensor, name: str) -> None:
        host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        host.copy_(ws[:4].view(torch.int32), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(ws.device))
        self.pending.append((ev, host, name))

    def poll(self, block: bool = False) -> None:
        while self.pending:
            ev, host, name = self.pending[0]
            if not block and len(self.pending) <= self.MAX_PENDING and not ev.query():
                return
            ev.synchronize()
            self.pending.popleft()
            _raise_for_status(int(host[0]), name)


_status_queue = _StatusQueue()


def _raise_for_status(status: int, name: str) -> None:
    if status & LS_ATTN_RING_TIMEOUT:
        raise RuntimeError(f"{name}: a wait for a staged K/V page expired; the output is invalid")
    if status:
        raise RuntimeError(f"{name}: unknown status {status:#x}")


def check_attn_status(ws: torch.Tensor, name: str, *, sync: bool = False) -> None:
    """Check an attention call's status word (the first 4 bytes of its workspace).

    By default the word is queued for a deferred, non-blocking check (see
    ``_StatusQueue``): earlier calls whose copies have landed are checked now,
    and this call is checked by a later poll.  With ``sync=True`` the host waits
    for the stream and raises at once if this call's wait for a staged page
    expired.  Under graph capture the word cannot be read; the call is then not
    checked here, and a replay whose wait expired shows it in its output instead
    (the rows of such a wave are NaN)."""
    if torch.cuda.is_current_stream_capturing():
        return
    if sync:
        _status_queue.poll(block=True)
        _raise_for_status(int(ws[:4].view(torch.int32).item()), name)
        return
    _status_queue.push(ws, name)
    _status_queue.poll(block=False)


def attn_status_sync() -> None:
    """Wait for every queued attention status word and raise for the first
    call whose wait for a staged K/V page expired."""
    _status_queue.poll(block=True)


def poll_attn_status() -> None:
    """Check the queued status words whose copies have landed (never waits)."""
    if not torch.cuda.is_current_stream_capturing():
        _status_queue.poll(block=False)


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
