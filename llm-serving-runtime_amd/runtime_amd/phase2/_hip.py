"""ctypes binding of libmxdecode.so (the C ABI declared in include/mxdecode.h).

The library is loaded lazily on first use. There is no fallback: if it is
missing or its ABI version differs, every entry point raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "libmxdecode.so")
ABI_VERSION = 18

MX_OK = 0
MX_ERR_INVALID = -1
MX_ERR_UNSUPPORTED = -2
MX_ERR_ALIGNMENT = -3
MX_ERR_NULL = -4
MX_ERR_LAUNCH = -5
MX_ERR_WORKSPACE = -6

_VALUE_ERRORS = {MX_ERR_INVALID, MX_ERR_UNSUPPORTED, MX_ERR_ALIGNMENT, MX_ERR_NULL, MX_ERR_WORKSPACE}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32

# name -> (restype, argtypes); mirrors include/mxdecode.h
SIGNATURES = {
    "mx_abi_version": (ctypes.c_int, []),
    "mx_last_error": (ctypes.c_char_p, []),
    "mx_w8a16_quantize": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _p]),
    "mx_w8a16_pack": (ctypes.c_int, [_p, _i64, _i64, _p, _p]),
    "mx_w8a16_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mx_w8a16_linear": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p, _sz, _p]),
    "mx_w8a16_splits": (ctypes.c_int, [_i64, _i64, _i64]),
    "mx_w8a16_linear_partials": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p, _i64, _p, _sz, _p]),
    "mx_w8a16_linear_swiglu": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p, _sz, _p]),
    "mx_w8a16_linear_partials_swiglu": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p, _i64, _p, _sz, _p]),
    "mx_w8a16_gateup_swiglu": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p]),
    "mx_w8a16_mlp_fused_supported": (ctypes.c_int, [_i64, _i64, _i64, _i64]),
    "mx_w8a16_mlp_fused_partials": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p, _p, _i64, _p, _i64, _p, _p, _i64, _p,
                                                   _sz, _p, _p]),
    "mx_paged_attn_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mx_paged_attn_error_offset": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mx_paged_attn_decode": (
        ctypes.c_int,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _i32, _i32, _i32, _i32, _i32, _i32,
         ctypes.c_float, _p, _i64, _i64, _p, _sz, _i32, _u32, _p],
    ),
    "mx_paged_attn_decode_noalloc": (
        ctypes.c_int,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _i32, _i32, _i32, _i32, _i32, _i32,
         ctypes.c_float, _p, _i64, _i64, _i32, _u32, _p, _p],
    ),
    "mx_kv_gather_probe": (
        ctypes.c_int, [_p, _p, _i64, _i64, _p, _i64, _i32, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p],
    ),
    "mx_kv_append": (
        ctypes.c_int,
        [_p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _p, _i64, _i32, _p, _p, _p, _i64, _i64, _i32, _i32, _p,
         _p, _p],
    ),
    "mx_qkv_rope_append": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _p, _i32, _p, _p, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _i32, _i32,
         _p, _p, _p, _p],
    ),
    "mx_add_rmsnorm": (
        ctypes.c_int,
        [_p, _i64, _p, _i64, _p, _i64, _p, _i32, _i32, ctypes.c_float, _p, _i64, _p, _i64, _p],
    ),
    "mx_argmax_rows": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p, _p]),
    "mx_argmax_workspace_bytes": (ctypes.c_size_t, [_i32, _i32]),
    "mx_argmax_rows_split": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p, _p, ctypes.c_size_t, _p]),
    "mx_swiglu_interleaved": (ctypes.c_int, [_p, _i64, _p, _i32, _p, _i32, _i32, _p, _i64, _p]),
    "mx_qkv_rope_append_splits": (
        ctypes.c_int,
        [_p, _i32, _p, _i32, _i32, _i32, _i32, _p, _i32, _p, _p, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _i32, _i32,
         _p, _p, _p, _p],
    ),
    "mx_w8a16_qkv_rope_append": (
        ctypes.c_int,
        [_p, _i64, _i64, _i64, _p, _p, _p, _i32, _i32, _i32, _p, _i32, _p, _p, _i64, _p, _p, _i64, _i64, _p, _i64,
         _i32, _i32, _i32, _p, _p, _p, _p],
    ),
    "mx_add_rmsnorm_splits": (
        ctypes.c_int,
        [_p, _i32, _p, _p, _i64, _p, _i32, _i32, ctypes.c_float, _p, _i64, _p, _i64, _p],
    ),
    "mx_silu_mul": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _i64, _p]),
    "mx_stream_probe": (ctypes.c_int, [_p, _i64, _i64, _i64, _i32, _i32, _p, _p]),
    "mx_launch_probe": (ctypes.c_int, [_p, _i64, _i64, _i32, _p]),
    "mx_run_gather_probe": (ctypes.c_int, [_p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _p]),
    "mx_handoff_probe": (ctypes.c_int, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _p]),
    "mx_barrier_probe": (ctypes.c_int, [_p, _i64, _p, _i64, _i32, _i32, _i32, _p, _p]),
    "mx_chain_probe": (ctypes.c_int, [_p, _i64, _i64, _i32, _i32, _i32, _i32, _p, _i64, _p, _i64, _p, _p, _p]),
}

_lib = None
_lock = threading.Lock()


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load libmxdecode.so and declare its prototypes (raises if unavailable)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libmxdecode.so not found at {LIB_PATH}; build it with "
                "`python llm-serving-runtime_amd/build.py` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.mx_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libmxdecode ABI version {version} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def available() -> bool:
    """True when the HIP library loads and a ROCm device is visible."""
    try:
        load()
    except (RuntimeError, OSError):
        return False
    return bool(torch.cuda.is_available() and torch.version.hip is not None)


def check(rc: int, what: str) -> None:
    if rc == MX_OK:
        return
    msg = load().mx_last_error().decode(errors="replace")
    if rc in _VALUE_ERRORS:
        raise ValueError(f"{what}: {msg} (status {rc})")
    raise RuntimeError(f"{what}: {msg} (status {rc})")


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def require_device_tensor(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a ROCm device tensor (got device {t.device}); this path has no CPU fallback")
