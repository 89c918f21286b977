"""ctypes binding of the C ABI declared in include/nanokv.h.

The shared library is loaded from this package directory.  There is no
fallback: if ``libnanokv.so`` is missing the first call raises, so a GPU run
can never silently take another path.
"""

from __future__ import annotations

import ctypes
import os

LIB_NAME = "libnanokv.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

NKV_OK = 0
NKV_ERR_ARG = 1
NKV_ERR_UNSUPPORTED = 2
NKV_ERR_HIP = 3

NKV_KV_BF16 = 0
NKV_KV_INT8_CHANNEL = 1
NKV_KV_INT8_TOKEN = 2

NKV_ORDER_SCORE_DESC = 0
NKV_ORDER_ID_ASC = 1

ABI_VERSION = 1


class NkvStore(ctypes.Structure):
    """Mirror of ``struct nkv_store``."""
    _fields_ = [
        ("hist_k", ctypes.c_void_p),
        ("hist_v", ctypes.c_void_p),
        ("reps", ctypes.c_void_p),
        ("sink_k", ctypes.c_void_p),
        ("sink_v", ctypes.c_void_p),
        ("recent_k", ctypes.c_void_p),
        ("recent_v", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("k_tscale", ctypes.c_void_p),
        ("v_tscale", ctypes.c_void_p),
        ("num_layers", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("r", ctypes.c_int32),
        ("cap_blocks", ctypes.c_int32),
        ("sink_tokens", ctypes.c_int32),
        ("recent_tokens", ctypes.c_int32),
        ("kv_format", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SP = ctypes.POINTER(NkvStore)

# name -> (restype, argtypes); the exported symbol set of include/nanokv.h
SIGNATURES = {
    "nkv_abi_version": (_I, []),
    "nkv_last_error": (ctypes.c_char_p, []),
    "nkv_select": (_I, [_SP, _I, _I, _P, _I64, _I, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P]),
    "nkv_attend": (_I, [_SP, _I, _I, _P, _I64, _I, _P, _P, _I64, _I, _I, _P, _I64, _I, _P, _I64,
                        _I, _I, _I, _I, _F, _I, _P, _P, _P]),
    "nkv_attend_workspace_floats": (_I64, [_I, _I, _I, _I, _I]),
    "nkv_set_attend_marks": (_I, [_P, _P]),
    "nkv_decode_step": (_I, [_SP, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F,
                             _I, _P, _P, _P, _P, _I, ctypes.POINTER(ctypes.c_void_p)]),
    "nkv_decode_step_workspace_floats": (_I64, [_I, _I, _I, _I, _I]),
    "nkv_rmsnorm": (_I, [_P, _P, _P, _P, _P, _I, _I, _F, _P]),
    "nkv_qk_norm_rope": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _I, _P, _F, _P, _P, _P, _P]),
    "nkv_silu_mul": (_I, [_P, _P, _I, _I, _P]),
    "nkv_gemv": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "nkv_gemv_silu_mul": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "nkv_decode_step_ring": (_I, [_SP, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _F, _I, _P, _P, _P,
                                  _P, _P]),
    "nkv_prefill_attend": (_I, [_SP, _I, _I, _P, _I64, _I, _P, _P, _I64, _P, _I64, _I, _P, _I64,
                                _I, _I, _I, _I, _F, _I, _P, _P, _P]),
    "nkv_prefill_workspace_floats": (_I64, [_I, _I, _I, _I, _I]),
    "nkv_select_union": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "nkv_select_per_query": (_I, [_SP, _I, _I, _P, _I64, _I, _I, _P, _I, _I, _P, _P, _P, _P, _I, _P, _P, _P,
                                  _P]),
    "nkv_store_chunk": (_I, [_SP, _I, _I, _P, _P, _I64, _I, _I, _I, _I, _P]),
    "nkv_build_reps": (_I, [_SP, _I, _I, _P, _I64, _I, _I, _P]),
    "nkv_recent_update": (_I, [_SP, _I, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _P]),
    "nkv_query_summaries": (_I, [_P, _I64, _I, _I, _I, _I, _I, _P, _I64, _P]),
    "nkv_host_device_pointer": (_I, [_P, ctypes.POINTER(ctypes.c_void_p)]),
    "nkv_attend_packed": (_I, [_I, _I, _P, _I, _P, _P, _I, _I, _P, _F, _I, _P, _P, _P]),
    "nkv_attend_packed_workspace_floats": (_I64, [_I, _I, _I, _I]),
    "nkv_prefill_attend_tiled": (_I, [_SP, _I, _I, _P, _I64, _I, _P, _P, _I64, _P, _I64, _I64, _I, _I, _I, _I,
                                      _I, _I, _F, _I, _P, _P, _P]),
    "nkv_decode_step_noalloc": (_I, [_SP, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F,
                                     _I, _P, _P, _P]),
}

_lib = None


def load():
    """Load libnanokv.so (raises RuntimeError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: the NanoKV HIP kernels are not built "
            "(run __graft_entry__.build()); there is no fallback path")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.nkv_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH}: ABI version {lib.nkv_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def host_device_pointer(host_ptr: int) -> int:
    """Device address of pinned host memory (nkv_host_device_pointer)."""
    lib = load()
    out = ctypes.c_void_p()
    check(lib.nkv_host_device_pointer(ctypes.c_void_p(host_ptr), ctypes.byref(out)),
          "host_device_pointer")
    return out.value


def set_attend_marks(before, after) -> None:
    """Record the hipEvent_t handles `before` / `after` (None: off) right before
    and right after the attention kernel of this thread's later attention
    launches (nkv_set_attend_marks): times the kernel apart from the
    selection before it and the split merge after it."""
    lib = load()
    check(lib.nkv_set_attend_marks(ctypes.c_void_p(before or None), ctypes.c_void_p(after or None)),
          "nkv_set_attend_marks")


def check(rc: int, what: str) -> None:
    """Map an nkv status code onto the reference's exception types."""
    if rc == NKV_OK:
        return
    msg = load().nkv_last_error().decode(errors="replace")
    if rc in (NKV_ERR_ARG, NKV_ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")
