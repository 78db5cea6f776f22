"""ctypes binding of ``libmoeinfra_hip.so`` (the gfx950 MoE expert-path kernels).

There is no fallback: if the library is missing or fails to load, :func:`lib` raises.
Build it with ``python -m moeinfra_amd.build``.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmoeinfra_hip.so")

MOE_STATUS_OK = 0
MOE_STATUS_INVALID_ARGUMENT = -1
MOE_STATUS_HIP_ERROR = -2
MOE_STATUS_UNSUPPORTED = -3
MOE_MAX_EXPERTS = 32
MOE_MAX_TOPK = 8
MOE_NF4_BLOCKSIZE = 64
MOE_NOALLOC_SCRATCH_BYTES = 64 << 20

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class MoeNf4Expert(ctypes.Structure):
    """Mirror of ``moe_nf4_expert_t`` (include/moeinfra_hip.h)."""

    _fields_ = [
        ("w1_packed", _vp), ("w1_absmax", _vp), ("w1_code", _vp),
        ("w3_packed", _vp), ("w3_absmax", _vp), ("w3_code", _vp),
        ("w2_packed", _vp), ("w2_absmax", _vp), ("w2_code", _vp),
    ]


#: Exported symbol -> (argtypes, restype).  tests/test_capi_symbols.py checks that this
#: table and include/moeinfra_hip.h declare the same entry points.
SIGNATURES = {
    "moe_last_error": ([], ctypes.c_char_p),
    "moe_version": ([], ctypes.c_int),
    "moe_wait_timeouts": ([ctypes.POINTER(_i64), _i32], ctypes.c_int),
    "moe_nf4_dequant_bf16": ([_vp, _vp, _vp, _vp, _i64, _i32, _vp], ctypes.c_int),
    "moe_nf4_quantize_bf16": ([_vp, _i64, _i32, _vp, _vp, _vp, _vp], ctypes.c_int),
    "moe_router_topk": ([_vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp],
                        ctypes.c_int),
    "moe_permute": ([_vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "moe_expert_ffn_nf4": ([ctypes.POINTER(MoeNf4Expert), _i32, _vp, _i64, _i32, _i32, _i32,
                            _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp], ctypes.c_int),
    "moe_expert_gateup_nf4": ([ctypes.POINTER(MoeNf4Expert), _i32, _vp, _i64, _i32, _i32, _i32,
                               _vp, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "moe_expert_down_nf4": ([ctypes.POINTER(MoeNf4Expert), _i32, _i64, _i32, _i32, _i32,
                             _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp], ctypes.c_int),
    "moe_combine": ([_vp, _i32, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _vp], ctypes.c_int),
    "moe_expert_workspace_bytes": ([_i64, _i32, _i32], ctypes.c_int64),
    "moe_expert_swiglu_nf4": ([ctypes.POINTER(MoeNf4Expert), _vp, _i64, _i32, _i32, _vp, _vp,
                               _i64, _vp], ctypes.c_int),
    "moe_layer_workspace_bytes": ([_i64, _i32, _i32, _i32, _i32], ctypes.c_int64),
    "moe_layer_down_splits": ([_i64, _i32, _i32, _i32, _i32], ctypes.c_int32),
    "moe_layer_forward_nf4": ([ctypes.POINTER(MoeNf4Expert), _i32, _vp, _vp, _vp, _i64, _i32,
                               _i32, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _vp], ctypes.c_int),
    "moe_layer_forward_nf4_noalloc": ([ctypes.POINTER(MoeNf4Expert), _i32, _vp, _vp, _vp, _i64,
                                       _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "moe_layer_forward_nf4_profiled": ([ctypes.POINTER(MoeNf4Expert), _i32, _vp, _vp, _vp, _i64,
                                        _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _i64,
                                        ctypes.POINTER(_vp), _vp], ctypes.c_int),
    "moe_add_rmsnorm_bf16": ([_vp, _vp, _vp, ctypes.c_float, _i64, _i32, _vp, _vp, _vp],
                             ctypes.c_int),
    "moe_rope_kv_bf16": ([_vp, _i64, _i32, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp],
                         ctypes.c_int),
    "moe_attention_bf16": ([_vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _i64, ctypes.c_float,
                            _vp, _vp], ctypes.c_int),
    "moe_gemv_bf16": ([_vp, _vp, _i64, _i32, _i32, _vp, _vp], ctypes.c_int),
    "moe_layer_norm_workspace_bytes": ([_i32, _i32, _i32, _i32], _i64),
    "moe_layer_forward_nf4_norm": ([ctypes.POINTER(MoeNf4Expert), _i32, _vp, _vp, _vp, _vp, ctypes.c_float, _i32, _i32, _i32,
                                    _vp, _vp, _vp, _vp, _vp, _i64, _vp], ctypes.c_int),
    "moe_nf4_expand_absmax": ([_vp, _vp, _vp, ctypes.c_float, _i64, _i32, _vp, _vp], ctypes.c_int),
    "moe_qkv_rope_bf16": ([_vp, _vp, _vp, _i64, _vp, _vp, ctypes.c_float, _i32, _i32, _i32, _i32,
                           _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "moe_head_argmax_bf16": ([_vp, _vp, _vp, _vp, ctypes.c_float, _i32, _i32, _vp, _vp, _i64, _vp,
                              _vp, _i64, _vp, _vp, _vp], ctypes.c_int),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MoeHipError(RuntimeError):
    """A HIP-side failure reported by libmoeinfra_hip."""


def lib() -> ctypes.CDLL:
    """Load the library once and declare its signatures.  Raises if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m moeinfra_amd.build` "
                    "(the MoE path has no non-HIP implementation)")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (argtypes, restype) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Map a C-ABI status to the reference's exception conventions."""
    if rc == MOE_STATUS_OK:
        return
    msg = (lib().moe_last_error() or b"").decode(errors="replace")
    if rc == MOE_STATUS_INVALID_ARGUMENT:
        raise ValueError(f"{what}: {msg}")
    if rc == MOE_STATUS_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise MoeHipError(f"{what}: {msg} (status {rc})")


def wait_timeouts(reset: bool = True) -> int:
    """Bounded in-kernel waits that gave up on the current device since the last reset
    (0 unless a kernel's wave counting went wrong).  Synchronous."""
    n = _i64(0)
    check(lib().moe_wait_timeouts(ctypes.byref(n), 1 if reset else 0), "moe_wait_timeouts")
    return int(n.value)
