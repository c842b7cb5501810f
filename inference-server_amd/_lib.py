"""ctypes binding of ``libmoe_mi355x.so`` (the C ABI in ``include/moe_mi355x.h``).

There is no fallback: if the library is missing or cannot be loaded, every op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libmoe_mi355x.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

_c_int, _c_size, _vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); mirrors include/moe_mi355x.h
SIGNATURES = {
    "moe_mi355x_error_string": (ctypes.c_char_p, [_c_int]),
    "moe_mi355x_version": (_c_int, []),
    "moe_mi355x_route_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "moe_mi355x_route": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp,
                                  _vp, _c_size, _vp]),
    "moe_mi355x_topk_softmax": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _c_int, _vp, _vp]),
    "moe_mi355x_align_max_tiles": (_c_int, [_c_int, _c_int, _c_int]),
    "moe_mi355x_align_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "moe_mi355x_align": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _c_size, _vp]),
    "moe_mi355x_quantize_act_fp8": (_c_int, [_vp, _c_int, _c_int, _vp, _vp, _vp]),
    "moe_mi355x_quantize_weight_fp8": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "moe_mi355x_experts_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "moe_mi355x_experts_fp8": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                        _vp, _vp, _vp, _vp, _c_size, _vp]),
    "moe_mi355x_block_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "moe_mi355x_block_fp8": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp,
                                      _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_size, _vp]),
    "moe_mi355x_experts_bf16_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "moe_mi355x_experts_bf16": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                         _vp, _vp, _c_size, _vp]),
    "moe_mi355x_block_bf16_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "moe_mi355x_block_bf16": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp,
                                       _vp, _c_int, _vp, _vp, _c_size, _vp]),
    "moe_mi355x_block_fp8_noalloc_scratch_bytes": (_c_size, []),
    "moe_mi355x_block_fp8_noalloc": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                              _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp]),
    "moe_mi355x_block_numerics_key": (ctypes.c_longlong, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "moe_mi355x_paged_attn_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "moe_mi355x_paged_attn_decode": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                              _c_int, _c_int, ctypes.c_float, _vp, _vp, _c_size, _vp]),
    "moe_mi355x_kv_append": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _vp]),
    "moe_mi355x_rms_norm": (_c_int, [_vp, _vp, _c_int, _c_int, ctypes.c_float, _vp, _vp]),
    "moe_mi355x_linear_bf16_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "moe_mi355x_linear_bf16": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_size, _vp]),
    "moe_mi355x_qk_norm_rope_append": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                                ctypes.c_float, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "moe_mi355x_moe_sublayer_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "moe_mi355x_moe_sublayer_fp8": (_c_int, [_vp, _vp, _vp, ctypes.c_float, _vp, _c_int, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "moe_mi355x_profile_enable": (_c_int, [_c_int]),
    "moe_mi355x_profile_read": (_c_int, [_c_int, ctypes.POINTER(_c_int), ctypes.POINTER(ctypes.c_double)]),
    "moe_mi355x_profile_slot_name": (ctypes.c_char_p, [_c_int]),
}

_lock = threading.Lock()
_lib = None


class MoEKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero code."""


# (major << 16) | minor of the C ABI these signatures describe (moe_mi355x_version)
ABI_VERSION = (0 << 16) | 2


def load() -> ctypes.CDLL:
    """Load the shared library once; raises ImportError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python inference-server_amd/build.py` "
                    "(or __graft_entry__.build()); there is no CPU fallback"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            got = lib.moe_mi355x_version()
            if got != ABI_VERSION:
                raise ImportError(f"{LIB_PATH} has ABI version {got >> 16}.{got & 0xFFFF}, this binding expects "
                                  f"{ABI_VERSION >> 16}.{ABI_VERSION & 0xFFFF}: rebuild it")
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().moe_mi355x_error_string(rc).decode()
        raise MoEKernelError(f"{what} failed with code {rc}: {msg}")
