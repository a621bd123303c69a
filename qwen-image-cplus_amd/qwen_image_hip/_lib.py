"""ctypes binding of libqwen_image_hip.so (the C ABI in include/qwen_image_hip.h).

The library is loaded from this directory only.  If it is missing the import
of any op fails loudly: there is no CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqwen_image_hip.so"

_i = ctypes.c_int
_p = ctypes.c_void_p
_u64 = ctypes.c_ulonglong

# name -> argtypes; restype is int (hipError_t) for all of them.
SIGNATURES: dict[str, list] = {
    "qi_hip_abi_version": [],
    "qi_w4a4_quantize_activations": [_p, _p, _p, _i, _i],
    "qi_w4a4_gemm": [_p, _p, _p, _p, _p, _i, _i, _i],
    "qi_w4a16_gemm": [_p, _p, _p, _p, _p, _i, _i, _i],
    "qi_f32_to_f16": [_p, _p, _u64],
    "qi_hip_w4a4_quantize_activations": [_p, _p, _p, _i, _i, _p],
    "qi_hip_f32_to_f16": [_p, _p, _u64, _p],
    "qi_hip_w4a4_quantize_activations_f16": [_p, _p, _p, _i, _i, _p],
    "qi_hip_relayout_w4a4": [_p, _p, _p, _p, _i, _i, _p],
    "qi_hip_relayout_w4a4_inverse": [_p, _p, _p, _p, _i, _i, _p],
    "qi_hip_relayout_w4a16": [_p, _p, _p, _p, _p, _i, _i, _p],
    "qi_hip_relayout_w4a16_inverse": [_p, _p, _p, _p, _p, _i, _i, _p],
    "qi_hip_w4a4_gemm_tiled": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "qi_hip_w4a16_gemm_tiled": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "qi_hip_w4a16_gemv": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "qi_hip_pack_weights": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "qi_hip_w4a4_quantize_activations_fp6": [_p, _i, _p, _p, _i, _i, _p],
    "qi_hip_relayout_w4a4_fp6": [_p, _p, _p, _p, _i, _i, _p],
    "qi_hip_w4a4_gemm_fp6": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "qi_hip_w4a4_gemm_fp6_parts": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p],
    "qi_hip_w4a4_gemm_fp6_dual": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p],
    "qi_hip_w4a16_gemm_tiled_parts": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p],
    "qi_hip_w4a16_gemm_tiled_dual": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p],
    "qi_hip_w4a16_tiles": [_i, _i],
    "qi_hip_w4a16_gemm_tiled_ws": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p, ctypes.c_longlong, _p],
    "qi_hip_w4a4_fp6_tiles": [_i, _i],
    "qi_flash_attention": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "qi_hip_flash_attention": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _p],
    "qi_hip_flash_attention_ws": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _p, ctypes.c_longlong, _p],
    "qi_hip_layer_norm_scale": [_p, _p, _i, _p, _i, _i, _i, _i, _p],
    "qi_hip_layer_norm_scale_quantize_fp6": [_p, _p, _i, _i, _p, _p, _i, _i, _p],
    "qi_hip_layer_norm_scale_quantize_fp6_noalloc": [_p, _p, _i, _i, _p, _i, _i, _p],
    "qi_hip_swiglu": [_p, _p, _p, _i, _u64, _p],
    "qi_hip_swiglu_quantize_fp6": [_p, _p, _p, _i, _i, _p],
    # QIPACK1 container (host I/O; QI_PACK_* status codes, not hipError_t).
    "qi_pack_open": [ctypes.c_char_p, _p],
    "qi_pack_info": [_p, _p, _p, _p, _p],
    "qi_pack_record_at": [_p, ctypes.c_uint32, _p],
    "qi_pack_find": [_p, ctypes.c_char_p],
    "qi_pack_read": [_p, _u64, _u64, _p],
    "qi_pack_verify": [_p, _i],
}
# Entry points whose return type is not int.
RESTYPES = {"qi_fnv1a": (_u64, [_u64, _p, _u64]), "qi_pack_close": (None, [_p]),
            "qi_hip_w4a16_workspace_bytes": (ctypes.c_longlong, [_i, _i, _i, _i]),
            "qi_hip_flash_attention_workspace_bytes": (ctypes.c_longlong, [_i, _i, _i])}

ABI_VERSION = 5

_lib = None


class QiHipError(RuntimeError):
    """A native entry point returned a non-zero hipError_t."""

    def __init__(self, what: str, status: int):
        # Same wording as the reference's ok() helper
        # (qwen_image_cuda/src/transformer.cplus:104-110), HIP instead of CUDA.
        super().__init__(f"hip linear: {what} failed (hip status {status})")
        self.status = status
        self.what = what


def load() -> ctypes.CDLL:
    """Load the in-tree library (once) and declare every entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python qwen-image-cplus_amd/build.py` "
            "(no CPU fallback exists for the HIP linear path)"
        )
    lib = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_LOCAL)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError = missing export
        fn.argtypes = args
        fn.restype = ctypes.c_int
    for name, (restype, args) in RESTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = restype
    if lib.qi_hip_abi_version() != ABI_VERSION:
        raise ImportError("libqwen_image_hip.so ABI version mismatch; rebuild it")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise QiHipError(what, status)
