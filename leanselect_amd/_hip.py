"""ctypes binding of ``libleanselect_hip.so`` (the C ABI in include/leanselect_hip.h).

The library is built in-tree by ``leanselect_amd.build``.  Loading fails loudly
when it is missing: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libleanselect_hip.so")

LS_F32, LS_BF16, LS_F16 = 0, 1, 2
LS_OK, LS_ERR_INVALID, LS_ERR_UNSUPPORTED, LS_ERR_WORKSPACE, LS_ERR_HIP = range(5)

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
    "ls_sparse_attn_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "ls_sparse_attn_varlen": (
        _i32, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _i32, _i64, _i64, _i32, _i32, _i32, _i32,
               _i32, _i32, _p, _i32, _i32, _f32, _i32, _p, _p, _p, _sz, _p]),
    "ls_cis_mean_pool": (
        _i32, [_p, _i64, _i64, _i32, _p, _i32, _i32, _i32, _i32, _i32, _p, _i32, _p]),
    "ls_page_maxpool_varlen": (
        _i32, [_p, _p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p,
               _p]),
    "ls_nosa_select_workspace_size": (
        _sz, [_i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "ls_nosa_select_prefill": (
        _i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _p, _i32, _i32, _i32,
               _i32, _i32, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
               _p, _i32, _p, _sz, _p]),
    "ls_nosa_attn_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "ls_nosa_attn_varlen": (
        _i32, [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i32, _p, _p, _i32, _i64, _i64, _i32,
               _i32, _i32, _i32, _i32, _i32, _p, _i32, _i32, _f32, _p, _p, _p, _sz, _p]),
    "ls_rmsnorm": (_i32, [_p, _i64, _p, _i64, _i32, _f32, _i32, _p, _i64, _p]),
    "ls_add_rmsnorm": (
        _i32, [_p, _i64, _p, _i64, _f32, _p, _i64, _i32, _f32, _i32, _p, _i64, _p]),
    "ls_rope_inplace": (
        _i32, [_p, _i64, _p, _i64, _i32, _i32, _i64, _i32, _p, _p, _i64, _i32, _p]),
    "ls_silu_mul": (_i32, [_p, _i64, _i64, _i32, _i32, _p, _i64, _p]),
    "ls_embed_scale": (_i32, [_p, _i64, _p, _i64, _i32, _f32, _i32, _p, _p]),
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


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
