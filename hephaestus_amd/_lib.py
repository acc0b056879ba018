"""ctypes binding of libhephfp8.so (the C ABI declared in include/hephfp8.h
and include/hephdecode.h).

The library is built in-tree by hephaestus_amd/build.py. There is no
fallback: if the shared object is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
import re

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhephfp8.so")
_INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
HEADERS = [os.path.join(_INCLUDE, "hephfp8.h"), os.path.join(_INCLUDE, "hephdecode.h")]

_lib = None

HEPH_OK = 0
HEPH_ERR_NULL = -1
HEPH_ERR_SHAPE = -2
HEPH_ERR_ALIGN = -3
HEPH_ERR_GROUP = -4
HEPH_ERR_DTYPE = -5
HEPH_ERR_WORKSPACE = -6
HEPH_ERR_FLAGS = -7
HEPH_ERR_DEVICE = -8
HEPH_ERR_LAUNCH = -9
HEPH_ERR_UNSUPPORTED = -10
HEPH_ERR_SCRATCH = -11

HEPH_DTYPE_BF16 = 0
HEPH_DTYPE_F32 = 1

FLAG_ADD_RESIDUAL = 0x1
FLAG_SKIP_QUANT = 0x2
FLAG_FORCE_GEMM = 0x8
FLAG_NO_FUSE = 0x10

SKINNY_MAX_M = 32



class LaunchOverrides(ctypes.Structure):
    """heph_launch_overrides: per-call launch-shape overrides (0 = built-in)."""
    _fields_ = [("gemv_ks", ctypes.c_int), ("gemv_waves", ctypes.c_int),
                ("gemv_u", ctypes.c_int), ("gemm_bm", ctypes.c_int),
                ("batch_split", ctypes.c_int), ("wide_tiles", ctypes.c_int),
                ("wide_waves", ctypes.c_int), ("split_spin_limit", ctypes.c_int),
                ("gemv_groups", ctypes.c_int), ("gemm_bn", ctypes.c_int)]


_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

SIGNATURES = {
    "heph_fp8_quant_act": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "heph_fp8_quant_weight": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "heph_fp8_linear": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _vp, _sz, _vp, _sz,
                             _i, _i, _i, _i, _i, _vp]),
    "heph_fp8_linear_with": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _vp, _sz, _vp, _sz,
                                  _i, _i, _i, _i, _i, _vp, ctypes.POINTER(LaunchOverrides)]),
    "heph_rmsnorm_quant_fp8": (_i, [_vp, _vp, _vp, _vp, _i, _i, ctypes.c_float, _i, _vp]),
    "heph_silu_mul_quant_fp8": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "heph_fp8_linear_noalloc": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "heph_noalloc_scratch_bytes": (_sz, []),
    "heph_fp8_linear_rmsnorm": (_i, [_vp, _i, _vp, _vp, ctypes.c_float, _vp, _vp, _i, _i, _vp,
                                     _sz, _vp, _sz, _i, _i, _i, _vp]),
    "heph_fp8_linear_swiglu": (_i, [_vp, _vp, _vp, ctypes.c_float, _vp, _vp, _i, _i, _vp, _sz,
                                    _vp, _sz, _i, _i, _vp]),
    "heph_bf16_linear": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "heph_fp8_q_ws_bytes": (_sz, [_i, _i]),
    "heph_fp8_s_ws_floats": (_sz, [_i, _i, _i]),
    "heph_fp8_linear_ws_bytes": (_sz, [_i, _i, _i]),
    "heph_strerror": (ctypes.c_char_p, [_i]),
    "heph_abi_version": (_i, []),
    "heph_profile_next_launch": (_i, [_vp, _vp]),
    "heph_last_kernel": (ctypes.c_char_p, []),
    # hephdecode.h
    "heph_embed_fp8": (_i, [_vp, _vp, _vp, _i, _vp, _i, _i, _i, _vp]),
    "heph_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, ctypes.c_float, _vp]),
    "heph_qk_norm_rope_kv": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                  ctypes.c_double, ctypes.c_float, _vp]),
    "heph_attention_ws_bytes": (_sz, [_i, _i]),
    "heph_attention_fp8kv": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "heph_rope_table_bf16": (_i, [_vp, _i, _i, ctypes.c_double, _vp]),
    "heph_attention_qkv_fp8kv": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i,
                                      _i, _i, ctypes.c_double, ctypes.c_float, _vp, _sz, _vp]),
    "heph_silu_mul": (_i, [_vp, _vp, _vp, _i, _vp]),
    "heph_argmax_ws_bytes": (_sz, [_i]),
    "heph_argmax_bf16": (_i, [_vp, _vp, _i, _vp, _sz, _vp]),
}

ATTN_MAX_KEYS = 262144
# HEPH_ABI_VERSION of include/hephfp8.h that these signatures follow
ABI_VERSION = 6


class HephLibraryMissing(ImportError):
    pass


def lib():
    """Load libhephfp8.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HephLibraryMissing(
                f"{LIB_PATH} not found: build it with `python hephaestus_amd/build.py` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        if L.heph_abi_version() != ABI_VERSION:
            raise HephLibraryMissing(
                f"{LIB_PATH} has ABI version {L.heph_abi_version()}, this binding follows "
                f"{ABI_VERSION}: rebuild it")
        _lib = L
    return _lib


def header_functions() -> list[str]:
    """Names of the functions include/hephfp8.h and hephdecode.h declare."""
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"\b(heph_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def strerror(status: int) -> str:
    return lib().heph_strerror(status).decode()
