"""ctypes binding of libnomas_moe.so (the C ABI in include/nomas_moe.h).

torch is imported first on purpose: its bundled HIP runtime
(libamdhip64.so.7) is then the one the library binds to, so device pointers
from torch's allocator and the library's own allocations live in one runtime.
There is no fallback: if the library is missing, loading fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

import torch  # noqa: F401  (must be loaded before the library, see above)

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# NOMAS_MOE_LIB selects another build of the same library (the sanitizer
# build, libnomas_moe_san.so, in the CPU tests)
LIB_PATH = os.environ.get("NOMAS_MOE_LIB") or os.path.join(_PKG_ROOT, "libnomas_moe.so")

_lib = None


class nomas_moe_config(C.Structure):
    _fields_ = [
        ("experts", C.c_int64),
        ("top_k", C.c_int64),
        ("shared_dense", C.c_double),
        ("seed", C.c_uint64),
    ]


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: the HIP library has not been built "
            "(run `make -C hy-nomas-rs_amd` or __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
    cfgp = C.POINTER(nomas_moe_config)
    hp = C.POINTER(vp)
    L.nomas_moe_config_validate.argtypes = [cfgp]
    L.nomas_moe_config_validate.restype = i32
    L.nomas_moe_from_random.argtypes = [cfgp, C.c_char_p, i64, i64, i32, C.c_uint64, i32, hp]
    L.nomas_moe_from_random.restype = i32
    L.nomas_moe_from_safetensors.argtypes = [cfgp, C.POINTER(C.c_char_p), i64, C.c_char_p, i64,
                                             i64, i32, i32, hp]
    L.nomas_moe_from_safetensors.restype = i32
    L.nomas_moe_from_host.argtypes = [cfgp, i64, i64, i32, i32] + [vp] * 13 + [hp]
    L.nomas_moe_from_host.restype = i32
    L.nomas_moe_forward.argtypes = [vp, vp, vp, i64, vp]
    L.nomas_moe_forward.restype = i32
    L.nomas_moe_forward_noalloc.argtypes = [vp, vp, vp, i64, vp]
    L.nomas_moe_forward_noalloc.restype = i32
    L.nomas_moe_forward_block.argtypes = [vp, vp, vp, i64, i64, vp, C.c_double, vp, vp, vp, vp]
    L.nomas_moe_forward_block.restype = i32
    L.nomas_moe_forward_host.argtypes = [vp, vp, vp, i64]
    L.nomas_moe_forward_host.restype = i32
    L.nomas_moe_n_params.argtypes = [vp]
    L.nomas_moe_n_params.restype = i64
    L.nomas_moe_routing.argtypes = [vp, vp, vp, vp, vp]
    L.nomas_moe_routing.restype = i32
    L.nomas_moe_dims.argtypes = [vp, vp, vp, vp, vp, vp]
    L.nomas_moe_dims.restype = i32
    L.nomas_moe_set_profiling.argtypes = [vp, i32]
    L.nomas_moe_set_profiling.restype = i32
    L.nomas_moe_stage_times.argtypes = [vp, vp]
    L.nomas_moe_stage_times.restype = i32
    L.nomas_moe_uses_mfma.argtypes = [vp]
    L.nomas_moe_uses_mfma.restype = i32
    L.nomas_moe_destroy.argtypes = [vp]
    L.nomas_moe_destroy.restype = None
    L.nomas_ffn_from_random.argtypes = [C.c_char_p, i64, i64, i32, C.c_uint64, i32, hp]
    L.nomas_ffn_from_random.restype = i32
    L.nomas_ffn_from_safetensors.argtypes = [C.POINTER(C.c_char_p), i64, C.c_char_p, i64, i64, i32,
                                             i32, hp]
    L.nomas_ffn_from_safetensors.restype = i32
    L.nomas_ffn_from_host.argtypes = [i64, i64, i32, i32] + [vp] * 6 + [hp]
    L.nomas_ffn_from_host.restype = i32
    L.nomas_ffn_forward.argtypes = [vp, vp, vp, i64, vp]
    L.nomas_ffn_forward.restype = i32
    L.nomas_ffn_forward_host.argtypes = [vp, vp, vp, i64]
    L.nomas_ffn_forward_host.restype = i32
    L.nomas_ffn_n_params.argtypes = [vp]
    L.nomas_ffn_n_params.restype = i64
    L.nomas_ffn_set_profiling.argtypes = [vp, i32]
    L.nomas_ffn_set_profiling.restype = i32
    L.nomas_ffn_stage_times.argtypes = [vp, vp]
    L.nomas_ffn_stage_times.restype = i32
    L.nomas_ffn_uses_mfma.argtypes = [vp]
    L.nomas_ffn_uses_mfma.restype = i32
    L.nomas_norm_modulate.argtypes = [i32, vp, vp, i64, i64, i64, vp, C.c_double, vp, vp, vp]
    L.nomas_norm_modulate.restype = i32
    L.nomas_gated_residual.argtypes = [i32, vp, vp, vp, vp, i64, i64, i64, vp]
    L.nomas_gated_residual.restype = i32
    L.nomas_ffn_destroy.argtypes = [vp]
    L.nomas_ffn_destroy.restype = None
    L.nomas_moe_last_error.argtypes = []
    L.nomas_moe_last_error.restype = C.c_char_p
    L.nomas_path_seed.argtypes = [C.c_uint64, C.c_char_p]
    L.nomas_path_seed.restype = C.c_uint64
    L.nomas_randn_affine.argtypes = [C.c_uint64, C.c_double, C.c_double, i64, vp]
    L.nomas_randn_affine.restype = None
    L.nomas_f32_to_bf16.argtypes = [vp, vp, i64]
    L.nomas_f32_to_bf16.restype = None
    L.nomas_f32_to_f16.argtypes = [vp, vp, i64]
    L.nomas_f32_to_f16.restype = None
    _lib = L
    return L


def last_error() -> str:
    return lib().nomas_moe_last_error().decode(errors="replace")
