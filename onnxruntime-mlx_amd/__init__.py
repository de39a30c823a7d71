"""MI355X execution provider for ONNX Runtime: host-side Python interface.

The compute path is libortmi_kernels.so (hand-written HIP for gfx950), reached here
through its C ABI with device pointers taken from torch tensors (torch is used for
device memory and streams only). The op functions mirror the reference EP's
operator surface for the int4-decoder path - same op names, attribute meanings and
error behaviour (an unsupported form raises, as the reference's claim/translate
errors do) - so callers and tests read like the reference's op tests.

There is no CPU fallback: if the kernel library is missing or no GPU is present,
every op raises.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
KERNEL_LIB = os.path.join(LIB_DIR, "libortmi_kernels.so")
EP_LIB = os.path.join(LIB_DIR, "libonnxruntime_mi355x_ep.so")

ORTMI_F32, ORTMI_F16, ORTMI_BF16 = 1, 10, 16

_kernels = None


class KernelError(RuntimeError):
    """A kernel-library call returned an error status."""


def kernel_library_path() -> str:
    return KERNEL_LIB


def load_kernels() -> ctypes.CDLL:
    """Load libortmi_kernels.so (raises if it has not been built)."""
    global _kernels
    if _kernels is None:
        if not os.path.exists(KERNEL_LIB):
            raise FileNotFoundError(
                f"{KERNEL_LIB} is missing: build it with onnxruntime-mlx_amd/build.py")
        lib = ctypes.CDLL(KERNEL_LIB)
        _declare(lib)
        _kernels = lib
    return _kernels


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# Exported C ABI (include/ortmi_kernels.h): name -> (restype, argtypes).
SIGNATURES = {
    "ortmi_abi_version": (ctypes.c_int, []),
    "ortmi_last_error": (ctypes.c_char_p, []),
    "ortmi_copy_small_h2d": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_void_p]),
    "ortmi_matmul_nbits": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                          _i32, _vp]),
    "ortmi_matmul_nbits_decode_fused": (ctypes.c_int, [
        _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp]),
    "ortmi_matmul_nbits_swiglu_pairs": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp]),
    "ortmi_matmul_nbits_decode_merge": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp]),
    "ortmi_decoder_decode_step_workspace_size": (_sz, [_vp]),
    "ortmi_decoder_decode_step": (ctypes.c_int, [
        _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
        _vp]),
    "ortmi_group_query_attention_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "ortmi_group_query_attention": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64,
        _i64, _i64, _i64, _f32, _i32, _i32, _vp, _sz, _vp]),
    "ortmi_group_query_attention_ex_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "ortmi_group_query_attention_ex": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _i64,
        _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _vp,
        _sz, _vp]),
    "ortmi_group_query_attention_sliding_workspace_size": (_sz, [_i64] * 6),
    "ortmi_group_query_attention_sliding": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _f32, _i64, _vp, _vp,
        _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _vp, _sz, _vp]),
    "ortmi_group_query_attention_noalloc_max_workspace": (_sz, []),
    "ortmi_group_query_attention_noalloc": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64,
        _i64, _i64, _i64, _f32, _i32, _i32, _vp]),
    "ortmi_group_query_attention_decode_capturable": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
        _f32, _i32, _i32, _vp, _sz, _vp]),
    "ortmi_group_query_attention_decode_splits": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "ortmi_group_query_attention_decode_partials": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
        _f32, _i32, _i32, _vp]),
    "ortmi_paged_attention_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "ortmi_paged_attention": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp,
        _i64, _i64, _i32, _i64, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _i64, _i64, _i64, _f32,
        _i32, _vp, _sz, _vp]),
    "ortmi_rotary_embedding": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _i64,
                                              _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    "ortmi_gather_block_quantized": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i64, _i64,
                                                    _i64, _i64, _i64, _i32, _vp]),
    "ortmi_rms_norm": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _vp]),
    "ortmi_gather_rows": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp]),
    "ortmi_swiglu": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _vp]),
    "ortmi_swiglu_pairs": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _vp]),
    "ortmi_binary": (ctypes.c_int, [_i32, _vp, _vp, _vp, _i64, _i32, _vp]),
    "ortmi_sigmoid": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp]),
    "ortmi_argmax_rows_workspace_size": (_sz, [_i64, _i64]),
    "ortmi_argmax_rows": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _vp, _sz, _vp]),
    "ortmi_argmax_axis": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp]),
    "ortmi_cast": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i64, _vp]),
}


def _declare(lib: ctypes.CDLL) -> None:
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def check(rc: int) -> None:
    if rc != 0:
        msg = load_kernels().ortmi_last_error().decode(errors="replace")
        raise KernelError(msg)


from . import ops  # noqa: E402  (ops needs the loader above)
from .ops import (  # noqa: E402,F401
    gather_block_quantized,
    group_query_attention,
    group_query_attention_decode_capturable,
    group_query_attention_sliding,
    matmul_nbits,
    paged_attention,
    rotary_embedding,
    simplified_layer_norm,
    skip_simplified_layer_norm,
)
