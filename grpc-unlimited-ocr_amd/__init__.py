"""Python binding of the MI355X (gfx950) rocm backend for grpc-unlimited-ocr's
fused layer ops.

The product is the C ABI in include/uocr_rocm.h, implemented by the
hand-written HIP kernels in csrc/ and built in-tree into
build/libuocr_rocm.so (`make` in this directory). This module loads that
library through ctypes and mirrors the reference's op set
(src/backend/cuda/ops.h:30-75, decode_ops.h:17-27) over torch tensors:
torch supplies device memory and the current stream, nothing else. There is
no fallback: if the library is not built, every op raises.

Errors follow the reference's convention (src/backend/cuda/context.cu:24-28,
decode_ops.cu:239): a rejected shape or argument raises ValueError (the
reference's std::invalid_argument) before anything is enqueued; a runtime or
launch failure raises RocmError (std::runtime_error), each with the C ABI's
"<what>: <detail>" message.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BUILD_DIR = os.path.join(HERE, "build")
LIB_PATH = os.path.join(BUILD_DIR, "libuocr_rocm.so")
HEADER_PATH = os.path.join(ROOT, "include", "uocr_rocm.h")

OK, INVALID_ARGUMENT, NO_DEVICE, RUNTIME_ERROR, LAUNCH_ERROR = 0, 1, 2, 3, 4
H2D, D2H, D2D = 1, 2, 3


class RocmError(RuntimeError):
    """A HIP runtime or launch failure reported by the C ABI."""


class StepState(ctypes.Structure):
    """uocr_rocm_step_state: same fields and order as the reference's
    uocr::cuda::StepState (src/backend/cuda/decode_ops.h:17-23)."""

    _fields_ = [
        ("token", ctypes.c_int64),
        ("pos", ctypes.c_int64),
        ("tok", ctypes.c_int64),
        ("page", ctypes.c_int64),
        ("query_page", ctypes.c_int64),
    ]


class RouteParams(ctypes.Structure):
    """uocr_rocm_route_params: the reference's RouteParams
    (src/backend/cuda/ops.h:112-120); defaults are Decoder::default_router's
    (src/model/decoder.cpp:58-62, src/model/block_router.h:16-26)."""

    _fields_ = [
        ("block_size", ctypes.c_int64),
        ("local_blocks", ctypes.c_int64),
        ("top_m", ctypes.c_int64),
        ("top_k", ctypes.c_int64),
        ("idx_scale", ctypes.c_float),
        ("floor", ctypes.c_float),
        ("sigma", ctypes.c_float),
    ]

    def __init__(self, block_size=32, local_blocks=4, top_m=16, top_k=12, idx_scale=None, floor=1e-4, sigma=1.0):
        import math

        scale = ctypes.c_float(128.0).value / ctypes.c_float(math.sqrt(128.0)).value if idx_scale is None else idx_scale
        super().__init__(block_size, local_blocks, top_m, top_k, scale, floor, sigma)


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int
_sz = ctypes.c_size_t

# argtypes of every entry point in include/uocr_rocm.h (restype is int unless
# stated otherwise).
_SIGNATURES = {
    "uocr_rocm_status_string": ([_int], ctypes.c_char_p),
    "uocr_rocm_last_error": ([], ctypes.c_char_p),
    "uocr_rocm_abi_version": ([], _int),
    "uocr_rocm_device_count": ([ctypes.POINTER(_int)], _int),
    "uocr_rocm_device_info": ([_int, ctypes.c_char_p, _sz, ctypes.POINTER(_int), ctypes.POINTER(_int),
                               ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], _int),
    "uocr_rocm_stream_create": ([_int, ctypes.POINTER(_vp)], _int),
    "uocr_rocm_stream_destroy": ([_vp], _int),
    "uocr_rocm_stream_synchronize": ([_vp], _int),
    "uocr_rocm_capture_begin": ([_vp], _int),
    "uocr_rocm_capture_end": ([_vp, ctypes.POINTER(_vp)], _int),
    "uocr_rocm_graph_launch": ([_vp, _vp], _int),
    "uocr_rocm_graph_destroy": ([_vp], _int),
    "uocr_rocm_malloc": ([ctypes.POINTER(_vp), _sz, _vp], _int),
    "uocr_rocm_free": ([_vp, _vp], _int),
    "uocr_rocm_host_alloc": ([ctypes.POINTER(_vp), _sz], _int),
    "uocr_rocm_host_free": ([_vp], _int),
    "uocr_rocm_memcpy": ([_vp, _vp, _sz, _int, _vp], _int),
    "uocr_rocm_zero": ([_vp, _sz, _vp], _int),
    "uocr_rocm_event_create": ([ctypes.POINTER(_vp)], _int),
    "uocr_rocm_event_destroy": ([_vp], _int),
    "uocr_rocm_event_record": ([_vp, _vp], _int),
    "uocr_rocm_event_elapsed_ms": ([_vp, _vp, ctypes.POINTER(_f32)], _int),
    "uocr_rocm_add_inplace": ([_vp, _vp, _vp, _i64], _int),
    "uocr_rocm_copy": ([_vp, _vp, _vp, _i64], _int),
    "uocr_rocm_rms_norm": ([_vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_layer_norm": ([_vp, _vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_gelu_erf": ([_vp, _vp, _i64], _int),
    "uocr_rocm_silu_mul": ([_vp, _vp, _vp, _i64], _int),
    "uocr_rocm_rope": ([_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64], _int),
    "uocr_rocm_gather_rows_bf16": ([_vp, _vp, _i64, _vp, _i64, _i64, _vp], _int),
    "uocr_rocm_gather_row_bf16": ([_vp, _vp, _i64, _i64, _i64, _vp], _int),
    "uocr_rocm_embed_step": ([_vp, _vp, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_rope_step": ([_vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_add_rms_norm": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_swiglu": ([_vp, _vp, _vp, _i64, _i64], _int),
    "uocr_rocm_rope_qk": ([_vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                           _i64], _int),
    "uocr_rocm_rope_qk_step": ([_vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_rms_norm_bf16": ([_vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_add_rms_norm_bf16": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_layer_norm_bf16": ([_vp, _vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_gelu_erf_bf16": ([_vp, _vp, _i64], _int),
    "uocr_rocm_swiglu_bf16": ([_vp, _vp, _vp, _i64, _i64], _int),
    "uocr_rocm_rope_bf16": ([_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64], _int),
    "uocr_rocm_rope_qk_bf16": ([_vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64,
                                _i64, _i64], _int),
    "uocr_rocm_rope_qk_step_bf16": ([_vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_gather_rows_bf16_bf16": ([_vp, _vp, _i64, _vp, _i64, _i64, _vp], _int),
    "uocr_rocm_embed_step_bf16": ([_vp, _vp, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_router_norm": ([_vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_router_norm_bf16": ([_vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_quick_gelu": ([_vp, _vp, _i64], _int),
    "uocr_rocm_quick_gelu_bf16": ([_vp, _vp, _i64], _int),
    "uocr_rocm_softmax_rows": ([_vp, _vp, _i64, _i64], _int),
    "uocr_rocm_scale_add_mask": ([_vp, _vp, _f32, _vp, _i64, _i64, _i64], _int),
    "uocr_rocm_gemv_bf16": ([_vp, _vp, _i64, _vp, _i64, _vp, _vp], _int),
    "uocr_rocm_linear": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp], _int),
    "uocr_rocm_linear_bf16x": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp], _int),
    "uocr_rocm_round_bf16": ([_vp, _vp, _i64, _vp], _int),
    "uocr_rocm_gelu_erf_to_bf16": ([_vp, _vp, _vp, _i64], _int),
    "uocr_rocm_layer_norm_to_bf16": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32], _int),
    "uocr_rocm_quick_gelu_to_bf16": ([_vp, _vp, _vp, _i64], _int),
    "uocr_rocm_linear_workspace_floats": ([_i64, _i64, _i64], _i64),
    "uocr_rocm_linear_ws": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i64], _int),
    "uocr_rocm_linear_bf16x_ws": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i64], _int),
    "uocr_rocm_linear_bf16x_add_ws": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i64], _int),
    "uocr_rocm_linear_bf16x_add_rows": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i64], _int),
    "uocr_rocm_linear_bf16x_gelu_erf_bf16": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp], _int),
    "uocr_rocm_linear_bf16x_quick_gelu_bf16": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp], _int),
    "uocr_rocm_gemm_nt": ([_vp, _i64, _i64, _i64, _f32, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64],
                          _int),
    "uocr_rocm_gemm_nn": ([_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64], _int),
    "uocr_rocm_gather_rows": ([_vp, _vp, _vp, _i64, _i64, _vp], _int),
    "uocr_rocm_scatter_add_rows": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64], _int),
    "uocr_rocm_im2col": ([_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp], _int),
    "uocr_rocm_im2col_bf16": ([_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp], _int),
    "uocr_rocm_chw_to_hwc": ([_vp, _vp, _i64, _i64, _i64, _vp], _int),
    "uocr_rocm_hwc_to_chw": ([_vp, _vp, _i64, _i64, _i64, _vp], _int),
    "uocr_rocm_concat_cols": ([_vp, _vp, _i64, _vp, _i64, _i64, _vp], _int),
    "uocr_rocm_attention": ([_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                             _i64, _i64, _f32, _vp, _i64], _int),
    "uocr_rocm_attention_rel_pos": ([_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _f32, _vp, _vp], _int),
    "uocr_rocm_attention_rel_pos_workspace_floats": ([_i64, _i64, _i64], _i64),
    "uocr_rocm_attention_rel_pos_windows_ws": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64,
                                                _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _vp,
                                                _vp, _vp, _i64], _int),
    "uocr_rocm_attention_bf16": ([_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                  _i64, _i64, _i64, _f32, _vp, _i64], _int),
    "uocr_rocm_attention_workspace_floats": ([_i64, _i64, _i64, _i64], _i64),
    "uocr_rocm_attention_ws": ([_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                                _i64, _i64, _f32, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_attention_bf16_ws": ([_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _f32, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_attention_masked_workspace_floats": ([_i64, _i64, _i64, _i64], _i64),
    "uocr_rocm_attention_masked_bf16_ws": ([_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                                            _i64, _i64, _i64, _i64, _f32, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_attention_rel_pos_windows_bf16_ws": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64,
                                                     _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                     _f32, _vp, _vp, _vp, _i64], _int),
    "uocr_rocm_attention_rel_pos_ws": ([_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                        _i64, _i64, _i64, _f32, _vp, _vp, _vp, _i64], _int),
    "uocr_rocm_split_heads": ([_vp, _vp, _i64, _i64, _i64, _i64, _vp], _int),
    "uocr_rocm_merge_heads": ([_vp, _vp, _i64, _i64, _i64, _vp], _int),
    "uocr_rocm_rel_pos_bias": ([_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp], _int),
    "uocr_rocm_rel_pos_softmax_rows": ([_vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp], _int),
    "uocr_rocm_append_step": ([_vp, _vp, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_append_step_bf16": ([_vp, _vp, _vp, _i64, _vp, _i64], _int),
    "uocr_rocm_attend_step_bf16": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp, _f32, _vp, _vp, _i64, _vp], _int),
    "uocr_rocm_attend_rope_kv_step_bf16": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _f32, _vp, _vp, _i64,
                                            _vp, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_attend_scratch_floats": ([_i64, _i64, _i64], _i64),
    "uocr_rocm_attend_step": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp, _f32, _vp, _vp, _i64, _vp], _int),
    "uocr_rocm_attend_step_noalloc": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp, _f32, _vp, _i64, _vp], _int),
    "uocr_rocm_block_summaries": ([_vp, _vp, _i64, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_summary_step": ([_vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_scores_step": ([_vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_route_blocks": ([_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64,
                                ctypes.POINTER(RouteParams), _vp], _int),
    "uocr_rocm_route_step": ([_vp, _vp, _i64, _vp, _vp, _i64, _vp, ctypes.POINTER(RouteParams), _vp], _int),
    "uocr_rocm_route_decode_step": ([_vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64,
                                     _vp, _vp, _i64, _vp, ctypes.POINTER(RouteParams), _i64, _vp, _vp, _vp], _int),
    "uocr_rocm_route_decode_step_segments": ([_vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _vp, _i64, _vp, _vp, _vp,
                                              _i64, _vp, _vp, _i64, _vp, ctypes.POINTER(RouteParams), _i64, _vp, _vp,
                                              _vp, _vp], _int),
    "uocr_rocm_scale_mask_softmax_rows": ([_vp, _vp, _f32, _vp, _i64, _i64, _i64], _int),
    "uocr_rocm_embed_add_rms_norm_step": ([_vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _f32], _int),
    "uocr_rocm_embed_add_rms_norm_step_bf16": ([_vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _f32], _int),
    "uocr_rocm_add_rms_norm_gemv_bf16": ([_vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _vp, _i64, _vp, _vp], _int),
    "uocr_rocm_add_rms_norm_swiglu_gemv_bf16": ([_vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _vp, _vp, _i64, _vp],
                                                _int),
    "uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16": ([_vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _vp, _vp, _i64, _vp,
                                                        _vp, _i64, _vp], _int),
    "uocr_rocm_attend_rope_kv_step": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _f32, _vp, _vp, _i64, _vp,
                                       _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_attend_segments_scratch_floats": ([_i64, _i64, _i64], _i64),
    "uocr_rocm_attend_rope_kv_step_segments": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _f32, _vp, _vp,
                                                _i64, _vp, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_attend_rope_kv_step_segments_bf16": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _f32, _vp,
                                                     _vp, _i64, _vp, _i64, _vp, _i64, _vp], _int),
    "uocr_rocm_attend_merge_gemv_bf16": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp], _int),
    "uocr_rocm_expert_topk": ([_vp, _vp, _i64, _i64, _i64, _vp, _vp], _int),
    "uocr_rocm_expert_scratch_floats": ([_i64, _i64], _i64),
    "uocr_rocm_expert_ffn_one": ([_vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp], _int),
    "uocr_rocm_gemv_f32": ([_vp, _vp, _i64, _vp, _i64, _vp, _vp], _int),
    "uocr_rocm_moe_ffn_one": ([_vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp,
                               _vp], _int),
}

_LIB: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """The loaded C ABI library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RocmError(f"{LIB_PATH} is not built: run `make` in {HERE} (or __graft_entry__.build())")
        # torch ships its own HIP runtime under the soname libamdhip64.so.7.
        # Loading torch first makes this library bind to that same runtime;
        # loaded the other way round, a process would hold two HIP runtimes
        # and torch's streams would be foreign handles here.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = handle
    return _LIB


def check(status: int) -> None:
    """Raise for a non-zero C ABI status, with the library's message."""
    if status == OK:
        return
    message = lib().uocr_rocm_last_error().decode()
    if status == INVALID_ARGUMENT:
        raise ValueError(message)
    raise RocmError(message)


def call(name: str, *args) -> None:
    """Call an entry point by name and raise on a non-zero status."""
    check(getattr(lib(), name)(*args))


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib().uocr_rocm_device_count(ctypes.byref(n)))
    return n.value


def device_info(index: int = 0) -> dict:
    name = ctypes.create_string_buffer(256)
    arch, cus = ctypes.c_int(0), ctypes.c_int(0)
    free_b, total_b = ctypes.c_uint64(0), ctypes.c_uint64(0)
    check(lib().uocr_rocm_device_info(index, name, 256, ctypes.byref(arch), ctypes.byref(cus), ctypes.byref(free_b),
                                      ctypes.byref(total_b)))
    return {"name": name.value.decode(), "gfx_arch": arch.value, "compute_units": cus.value,
            "free_bytes": free_b.value, "total_bytes": total_b.value}


# ---- torch plumbing -----------------------------------------------------------


def _torch():
    import torch  # imported lazily: the CPU-side tests need only ctypes

    return torch


def current_stream() -> int:
    """torch's current stream on the current device, as the C ABI takes it."""
    return _torch().cuda.current_stream().cuda_stream


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr()


def _is_bf16(t) -> bool:
    torch = _torch()
    if t.dtype == torch.bfloat16:
        return True
    if t.dtype == torch.float32:
        return False
    raise ValueError(f"activations must be float32 or bfloat16, got {t.dtype}")


def _rows_cols(x):
    if x.dim() < 1:
        raise ValueError("tensor must have at least one axis")
    cols = x.shape[-1]
    return (x.numel() // cols if cols else 0), cols


def _f32_param(t):
    torch = _torch()
    if t is not None and t.dtype != torch.float32:
        raise ValueError("norm weights, biases and rope tables are float32")
    return _ptr(t)


def _op(name: str, stream, *args) -> None:
    """Call op `name` on `stream` (torch's current stream when None). The
    stream is resolved after the other arguments have been checked."""
    call(name, current_stream() if stream is None else stream, *args)


# ---- ops (mirroring uocr::cuda / uocr::rocm) -------------------------------------


def add_inplace(y, x, stream=None):
    """y += x (fp32). Reference: add_inplace, src/backend/cuda/ops.h:30."""
    _op("uocr_rocm_add_inplace", stream, _ptr(y), _ptr(x), y.numel())


def copy(dst, src, stream=None):
    """dst = src (fp32, device to device). Reference: copy, ops.h:68-69."""
    _op("uocr_rocm_copy", stream, _ptr(dst), _ptr(src), src.numel())


def rms_norm(x, w, eps, stream=None):
    """In place over the rows of x (fp32 or bf16). Reference: rms_norm, ops.h:34."""
    rows, cols = _rows_cols(x)
    name = "uocr_rocm_rms_norm_bf16" if _is_bf16(x) else "uocr_rocm_rms_norm"
    _op(name, stream, _ptr(x), _f32_param(w), rows, cols, eps)


def add_rms_norm(x, delta, w, h, eps, stream=None):
    """x += delta; h = rms_norm(x) * w, fused (fp32 or bf16)."""
    rows, cols = _rows_cols(x)
    bf = _is_bf16(x)
    if _is_bf16(delta) != bf or _is_bf16(h) != bf:
        raise ValueError("x, delta and h must share a dtype")
    if delta.numel() != x.numel() or h.numel() != x.numel():
        raise ValueError("x, delta and h must have the same shape")
    _op("uocr_rocm_add_rms_norm_bf16" if bf else "uocr_rocm_add_rms_norm", stream, _ptr(x), _ptr(delta),
         _f32_param(w), _ptr(h), rows, cols, eps)


def layer_norm(x, w, b, eps, stream=None):
    """In place over the rows of x (fp32 or bf16). Reference: layer_norm, ops.h:32-33."""
    rows, cols = _rows_cols(x)
    name = "uocr_rocm_layer_norm_bf16" if _is_bf16(x) else "uocr_rocm_layer_norm"
    _op(name, stream, _ptr(x), _f32_param(w), _f32_param(b), rows, cols, eps)


def gelu_erf(x, stream=None):
    """In place exact GELU (fp32 or bf16). Reference: gelu_erf, ops.h:37."""
    name = "uocr_rocm_gelu_erf_bf16" if _is_bf16(x) else "uocr_rocm_gelu_erf"
    _op(name, stream, _ptr(x), x.numel())


def silu_mul(g, u, stream=None):
    """g = silu(g) * u (fp32). Reference: silu_mul, ops.h:39."""
    _op("uocr_rocm_silu_mul", stream, _ptr(g), _ptr(u), g.numel())


def swiglu(inp, out, stream=None):
    """out [rows, F] = silu(inp[:, :F]) * inp[:, F:] for inp [rows, 2F]."""
    rows, two_f = _rows_cols(inp)
    if two_f % 2:
        raise ValueError("swiglu input width must be 2 * ffn")
    bf = _is_bf16(inp)
    if _is_bf16(out) != bf or out.numel() != rows * (two_f // 2):
        raise ValueError("swiglu output must be [rows, ffn] of the input's dtype")
    _op("uocr_rocm_swiglu_bf16" if bf else "uocr_rocm_swiglu", stream, _ptr(inp), _ptr(out), rows, two_f // 2)


def rope(x, heads, dim, tok, page, inv_tok, inv_page, page_mod, one_tok=0, one_page=0, stream=None):
    """In place rope on x [rows, heads * dim] (fp32 or bf16). Reference: rope, ops.h:48-52."""
    rows = x.numel() // (heads * dim) if heads * dim else 0
    n_tok = 0 if inv_tok is None else inv_tok.numel()
    n_page = 0 if inv_page is None else inv_page.numel()
    name = "uocr_rocm_rope_bf16" if _is_bf16(x) else "uocr_rocm_rope"
    _op(name, stream, _ptr(x), rows, heads, dim, _ptr(tok), _ptr(page), _f32_param(inv_tok), n_tok,
         _f32_param(inv_page), n_page, page_mod, one_tok, one_page)


def rope_qk(q, q_heads, k, k_heads, dim, tok, page, inv_tok, inv_page, page_mod, one_tok=0, one_page=0, stream=None):
    """rope on Q [rows, q_heads * dim] and K [rows, k_heads * dim] in one launch."""
    rows = q.numel() // (q_heads * dim) if q_heads * dim else k.numel() // (k_heads * dim)
    bf = _is_bf16(q)
    if k is not None and _is_bf16(k) != bf:
        raise ValueError("q and k must share a dtype")
    if k is not None and k_heads and k.numel() != rows * k_heads * dim:
        raise ValueError("k must have the rows of q")
    n_tok = 0 if inv_tok is None else inv_tok.numel()
    n_page = 0 if inv_page is None else inv_page.numel()
    _op("uocr_rocm_rope_qk_bf16" if bf else "uocr_rocm_rope_qk", stream, _ptr(q), q_heads, _ptr(k), k_heads,
         rows, dim, _ptr(tok), _ptr(page), _f32_param(inv_tok), n_tok, _f32_param(inv_page), n_page, page_mod,
         one_tok, one_page)


def rope_qk_step(q, q_heads, k, k_heads, dim, state, inv_tok, inv_page, page_mod, stream=None):
    """rope_qk of one decode row at the device StepState `state` (an int64 tensor of 5)."""
    n_tok = 0 if inv_tok is None else inv_tok.numel()
    name = "uocr_rocm_rope_qk_step_bf16" if _is_bf16(q) else "uocr_rocm_rope_qk_step"
    _op(name, stream, _ptr(q), q_heads, _ptr(k), k_heads, dim, _ptr(state), _f32_param(inv_tok), n_tok,
         _f32_param(inv_page), page_mod)


def gather_rows_bf16(table, index, out, table_rows=None, stream=None):
    """out[r] = table[index[r]] for a bf16 table; out is float32 (widened) or
    bfloat16 (bit copy). Reference: gather_rows_bf16, ops.h:72-73."""
    rows, cols = out.shape[0], table.shape[-1]
    bound = table.shape[0] if table_rows is None else table_rows
    name = "uocr_rocm_gather_rows_bf16_bf16" if _is_bf16(out) else "uocr_rocm_gather_rows_bf16"
    _op(name, stream, _ptr(table), bound, _ptr(index), rows, cols, _ptr(out))


def gather_row_bf16(table, one_index, out, stream=None):
    """out = widen(table[one_index]). Reference: gather_row_bf16, ops.h:74-75."""
    _op("uocr_rocm_gather_row_bf16", stream, _ptr(table), table.shape[0], one_index, table.shape[-1], _ptr(out))


def embed_step(table, state, out, stream=None):
    """out = table[state.token] read on the device. Reference: embed_step, decode_ops.h:25."""
    name = "uocr_rocm_embed_step_bf16" if _is_bf16(out) else "uocr_rocm_embed_step"
    _op(name, stream, _ptr(table), table.shape[0], _ptr(state), table.shape[-1], _ptr(out))


def rope_inv(n: int, theta: float):
    """PageRope's frequency table (src/model/page_rope.cpp:17-19):
    float32(1 / theta ** (i / n)) evaluated in float64, i < n."""
    import numpy as np

    i = np.arange(n, dtype=np.float64)
    return (1.0 / np.power(np.float64(theta), i / np.float64(n))).astype(np.float32)


# ---- row ops beside the path ---------------------------------------------------------


def router_norm(x, w, eps, stream=None):
    """In place router norm over the rows of x (fp32 or bf16): non-finite
    inputs zeroed, scaled by (1 + w), clamped to +-1e4. Reference:
    router_norm, src/backend/cuda/ops.h:35-36."""
    rows, cols = _rows_cols(x)
    name = "uocr_rocm_router_norm_bf16" if _is_bf16(x) else "uocr_rocm_router_norm"
    _op(name, stream, _ptr(x), _f32_param(w), rows, cols, eps)


def quick_gelu(x, stream=None):
    """In place x * sigmoid(1.702 x) (fp32 or bf16). Reference: quick_gelu, ops.h:38."""
    name = "uocr_rocm_quick_gelu_bf16" if _is_bf16(x) else "uocr_rocm_quick_gelu"
    _op(name, stream, _ptr(x), x.numel())


def softmax_rows(x, stream=None):
    """In place softmax over each row of x (fp32); all -inf rows become zeros.
    Reference: softmax_rows, ops.h:41-43."""
    if _is_bf16(x):
        raise ValueError("softmax_rows takes float32")
    rows, cols = _rows_cols(x)
    _op("uocr_rocm_softmax_rows", stream, _ptr(x), rows, cols)


def scale_add_mask(x, scale, mask, batch, rows, cols, stream=None):
    """x[b, r, c] = x[b, r, c] * scale + mask[r, c] (fp32; mask may be None).
    Reference: scale_add_mask, ops.h:44-46."""
    if _is_bf16(x):
        raise ValueError("scale_add_mask takes float32")
    if x.numel() != batch * rows * cols or (mask is not None and mask.numel() != rows * cols):
        raise ValueError("x must hold batch * rows * cols and mask rows * cols elements")
    _op("uocr_rocm_scale_add_mask", stream, _ptr(x), scale, _f32_param(mask), batch, rows, cols)


def scale_mask_softmax_rows(x, scale, mask, batch, rows, cols, stream=None):
    """x[b, r] = softmax(x[b, r] * scale + mask[r]) in one pass (fp32; mask may
    be None); bitwise scale_add_mask then softmax_rows."""
    if _is_bf16(x):
        raise ValueError("scale_mask_softmax_rows takes float32")
    if x.numel() != batch * rows * cols or (mask is not None and mask.numel() != rows * cols):
        raise ValueError("x must hold batch * rows * cols and mask rows * cols elements")
    _op("uocr_rocm_scale_mask_softmax_rows", stream, _ptr(x), scale, _f32_param(mask), batch, rows, cols)


# ---- decode-step neighbours ---------------------------------------------------------------


def gemv_bf16(x, w, y, bias=None, stream=None):
    """y[n] = bf16(x) . w[n] (+ bias): x float32 [k], w bfloat16 [n, k], y
    float32 [n]. Reference: gemv_bf16, src/backend/cuda/gemv_ops.h:25-26."""
    torch = _torch()
    if w.dtype != torch.bfloat16 or x.dtype != torch.float32 or y.dtype != torch.float32:
        raise ValueError("gemv_bf16 takes float32 x and y and bfloat16 w")
    n, k = w.shape
    if x.numel() != k or y.numel() != n or (bias is not None and bias.numel() != n):
        raise ValueError("gemv_bf16 shapes: x [k], w [n, k], y [n], bias [n]")
    _op("uocr_rocm_gemv_bf16", stream, _ptr(x), k, _ptr(w), n, _f32_param(bias), _ptr(y))


def linear_workspace_floats(m, k, n):
    """Workspace floats linear_ws would split k over (0: no split taken)."""
    return int(lib().uocr_rocm_linear_workspace_floats(m, k, n))


def linear_ws(x, w, y, workspace, bias=None, stream=None):
    """linear with a workspace for splitting k (new)."""
    torch = _torch()
    n, k = w.shape
    m = x.numel() // k
    name = "uocr_rocm_linear_bf16x_ws" if x.dtype == torch.bfloat16 else "uocr_rocm_linear_ws"
    _op(name, stream, _ptr(x), m, k, _ptr(w), n, _f32_param(bias), _ptr(y), _ptr(workspace), workspace.numel())


def linear_add(x, w, y, workspace, bias=None, stream=None):
    """y += bf16 x [m, k] . w[n, k]^T (+ bias) (new: a residual stream's
    projection, bitwise linear into a temporary then add_inplace)."""
    n, k = w.shape
    m = x.numel() // k
    _op("uocr_rocm_linear_bf16x_add_ws", stream, _ptr(x), m, k, _ptr(w), n, _f32_param(bias), _ptr(y),
        _ptr(workspace), workspace.numel())


def linear_add_rows(x, w, y, y_row, bias=None, stream=None):
    """y[y_row[r]] += (bf16 x . w^T + bias)[r], rows mapping to y.shape[0] or
    more dropped (new: window slots added back into their grid rows)."""
    n, k = w.shape
    m = x.numel() // k
    _op("uocr_rocm_linear_bf16x_add_rows", stream, _ptr(x), m, k, _ptr(w), n, _f32_param(bias), _ptr(y), _ptr(y_row),
        y.shape[0])


def linear_act(x, w, y, bias=None, quick=False, stream=None):
    """y = bf16(gelu_erf(bf16 x [m, k] . w[n, k]^T + bias)) (quick:
    quick_gelu), y bfloat16 [m, n] (new: an MLP's first projection with its
    activation and the rounding its second projection applies, bitwise
    linear then act_to_bf16)."""
    n, k = w.shape
    m = x.numel() // k
    if y.numel() != m * n:
        raise ValueError("linear_act: y [m, n]")
    name = "uocr_rocm_linear_bf16x_quick_gelu_bf16" if quick else "uocr_rocm_linear_bf16x_gelu_erf_bf16"
    _op(name, stream, _ptr(x), m, k, _ptr(w), n, _f32_param(bias), _ptr(y))


def linear(x, w, y, bias=None, stream=None):
    """y[m, n] = bf16(x)[m, k] . w[n, k]^T (+ bias[n]) on the matrix cores,
    fp32 accumulation: x float32 [m, k], w bfloat16 [n, k], y float32 [m, n].
    Reference: linear, src/backend/cuda/ops.h:14-17."""
    torch = _torch()
    if w.dtype != torch.bfloat16 or x.dtype not in (torch.float32, torch.bfloat16) or y.dtype != torch.float32:
        raise ValueError("linear takes float32 (or already rounded bfloat16) x, float32 y and bfloat16 w")
    n, k = w.shape
    m = x.numel() // k if k else 0
    if x.numel() != m * k or y.numel() != m * n or (bias is not None and bias.numel() != n):
        raise ValueError("linear shapes: x [m, k], w [n, k], y [m, n], bias [n]")
    if not (x.is_contiguous() and w.is_contiguous() and y.is_contiguous()):
        raise ValueError("linear takes contiguous x, w and y")
    name = "uocr_rocm_linear_bf16x" if x.dtype == torch.bfloat16 else "uocr_rocm_linear"
    _op(name, stream, _ptr(x), m, k, _ptr(w), n, _f32_param(bias), _ptr(y))


def round_bf16(src, dst, stream=None):
    """dst = bf16(src), nearest even (float32 -> bfloat16 tensors)."""
    if src.numel() != dst.numel():
        raise ValueError("round_bf16: src and dst sizes differ")
    _op("uocr_rocm_round_bf16", stream, _ptr(src), src.numel(), _ptr(dst))


def layer_norm_to_bf16(x, w, b, y, eps, stream=None):
    """y = bf16(layer_norm(x)) out of place: x float32 [rows, cols] untouched,
    y bfloat16 of the same shape (new: a LayerNorm read only by a
    projection, with the projection's rounding)."""
    cols = w.numel()
    if x.numel() != y.numel() or b.numel() != cols or (cols and x.numel() % cols):
        raise ValueError("layer_norm_to_bf16: x and y [rows, cols], w and b [cols]")
    rows = x.numel() // cols if cols else 0
    _op("uocr_rocm_layer_norm_to_bf16", stream, _ptr(x), _ptr(w), _ptr(b), _ptr(y), rows, cols, float(eps))


def act_to_bf16(x, y, quick=False, stream=None):
    """y = bf16(gelu_erf(x)) (quick: bf16(quick_gelu(x))), x float32 and y
    bfloat16 of the same size (new: an MLP's activation with the rounding its
    second projection applies)."""
    if x.numel() != y.numel():
        raise ValueError("act_to_bf16: x and y sizes differ")
    name = "uocr_rocm_quick_gelu_to_bf16" if quick else "uocr_rocm_gelu_erf_to_bf16"
    _op(name, stream, _ptr(x), _ptr(y), x.numel())


def gemm_nt(m, n, k, alpha, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch=1, stream=None):
    """c[s] = alpha a[s] . b[s]^T over `batch` slices (fp32 tensors, leading
    dimensions and slice strides in elements). Reference: gemm_nt,
    src/backend/cuda/ops.h:19-25."""
    _op("uocr_rocm_gemm_nt", stream, m, n, k, alpha, _ptr(a), lda, stride_a, _ptr(b), ldb, stride_b, _ptr(c), ldc,
        stride_c, batch)


def gemm_nn(m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch=1, stream=None):
    """c[s] = a[s] . b[s] over `batch` slices (fp32). Reference: gemm_nn,
    src/backend/cuda/ops.h:26-27."""
    _op("uocr_rocm_gemm_nn", stream, m, n, k, _ptr(a), lda, stride_a, _ptr(b), ldb, stride_b, _ptr(c), ldc, stride_c,
        batch)


def gather_rows(src, index, dst, stream=None):
    """dst[i] = src[index[i]] (fp32 rows). Reference: gather_rows, ops.h:56-57."""
    rows, cols = index.numel(), src.shape[-1]
    _op("uocr_rocm_gather_rows", stream, _ptr(src), _ptr(index), rows, cols, _ptr(dst))


def scatter_add_rows(dst, index, weight, src, stream=None):
    """dst[index[i]] += weight[i] * src[i], i in order. Reference:
    scatter_add_rows, ops.h:58-59."""
    rows, cols = index.numel(), dst.shape[-1]
    _op("uocr_rocm_scatter_add_rows", stream, _ptr(dst), _ptr(index), _ptr(weight), _ptr(src), rows, cols)


def im2col(x, kh, kw, stride, pad, cols, stream=None):
    """cols [oh * ow, c * kh * kw] = the patches of x [c, h, w] in weight
    order. Reference: im2col, ops.h:54-56."""
    c, h, w = x.shape
    # a bfloat16 cols: the patches rounded to bf16 (new)
    name = "uocr_rocm_im2col_bf16" if cols.dtype == _torch().bfloat16 else "uocr_rocm_im2col"
    _op(name, stream, _ptr(x), c, h, w, kh, kw, stride, pad, _ptr(cols))


def chw_to_hwc(x, y, stream=None):
    """y [h, w, c] = x [c, h, w]. Reference: chw_to_hwc, ops.h:57."""
    c, h, w = x.shape
    _op("uocr_rocm_chw_to_hwc", stream, _ptr(x), c, h, w, _ptr(y))


def hwc_to_chw(x, y, stream=None):
    """y [c, h, w] = x [h, w, c]. Reference: hwc_to_chw, ops.h:58."""
    h, w, c = x.shape
    _op("uocr_rocm_hwc_to_chw", stream, _ptr(x), h, w, c, _ptr(y))


def concat_cols(a, b, out, stream=None):
    """out[r] = a[r] | b[r]. Reference: concat_cols, ops.h:65-67."""
    _op("uocr_rocm_concat_cols", stream, _ptr(a), a.shape[-1], _ptr(b), b.shape[-1], a.shape[0], _ptr(out))


def _operand(t, offset, ld, slice_stride):
    return (_ptr(t) + t.element_size() * offset, ld, slice_stride)


def attention(q, k, v, out, slices, rows, keys, hd, scale, mask=None, strides=None, workspace=None, stream=None):
    """out[s, t] = softmax(scale q[s, t] . k[s, :] + mask[t, :]) v[s, :] in one
    pass (new). strides: {name: (offset, ld, slice_stride)} for q, k, v, out
    (elements); default head-major [slices, rows or keys, hd]. workspace
    (attention_workspace_floats floats): a mask's live tiles walked alone,
    long walks cut into runs merged by a last launch."""
    st = strides or {}
    qo = _operand(q, *st.get("q", (0, hd, rows * hd)))
    ko = _operand(k, *st.get("k", (0, hd, keys * hd)))
    vo = _operand(v, *st.get("v", (0, hd, keys * hd)))
    oo = _operand(out, *st.get("out", (0, hd, rows * hd)))
    # a bfloat16 out: the output rounded to bf16 in the epilogue (new)
    name = "uocr_rocm_attention_bf16" if out.dtype == _torch().bfloat16 else "uocr_rocm_attention"
    args = (*qo, *ko, *vo, *oo, slices, rows, keys, hd, scale, _f32_param(mask), 0 if mask is None else mask.shape[-1])
    if workspace is None:
        _op(name, stream, *args)
    else:
        _op(name + "_ws", stream, *args, _ptr(workspace), workspace.numel())


def attention_workspace_floats(slices, rows, keys, hd):
    """Floats of attention's workspace for a mask."""
    return int(lib().uocr_rocm_attention_workspace_floats(slices, rows, keys, hd))


def attention_masked(q, k, v, out, slices, rows, keys, hd, scale, mask, workspace, strides=None, stream=None):
    """attention with a mask into a bfloat16 out on the bf16 matrix cores,
    each fp32 operand split into bf16 hi + lo parts (new); workspace holds
    attention_masked_workspace_floats(slices, rows, keys, hd) floats (the
    mask's live tiles and the split key and value tiles). Strides as for
    attention."""
    if out.dtype != _torch().bfloat16:
        raise ValueError("attention_masked writes a bfloat16 out")
    st = strides or {}
    qo = _operand(q, *st.get("q", (0, hd, rows * hd)))
    ko = _operand(k, *st.get("k", (0, hd, keys * hd)))
    vo = _operand(v, *st.get("v", (0, hd, keys * hd)))
    oo = _operand(out, *st.get("out", (0, hd, rows * hd)))
    _op("uocr_rocm_attention_masked_bf16_ws", stream, *qo, *ko, *vo, *oo, slices, rows, keys, hd, scale, _ptr(mask),
        mask.shape[-1], _ptr(workspace), workspace.numel())


def attention_masked_workspace_floats(slices, rows, keys, hd):
    """Floats of attention_masked's workspace."""
    return int(lib().uocr_rocm_attention_masked_workspace_floats(slices, rows, keys, hd))


def attention_rel_pos(q, k, v, out, slices, h, w, hd, scale, rh, rw, strides=None, workspace=None, stream=None):
    """attention over h x w windows with SAM's relative-position bias (new);
    with a workspace (attention_rel_pos_workspace_floats) the bias's dot
    products are formed by a launch of their own first."""
    n = h * w
    st = strides or {}
    qo = _operand(q, *st.get("q", (0, hd, n * hd)))
    ko = _operand(k, *st.get("k", (0, hd, n * hd)))
    vo = _operand(v, *st.get("v", (0, hd, n * hd)))
    oo = _operand(out, *st.get("out", (0, hd, n * hd)))
    if workspace is None:
        _op("uocr_rocm_attention_rel_pos", stream, *qo, *ko, *vo, *oo, slices, h, w, hd, scale, _ptr(rh), _ptr(rw))
    else:
        _op("uocr_rocm_attention_rel_pos_ws", stream, *qo, *ko, *vo, *oo, slices, h, w, hd, scale, _ptr(rh),
            _ptr(rw), _ptr(workspace), workspace.numel())


def attention_rel_pos_windows(qkv, out, heads, windows, h, w, hd, scale, rh, rw, workspace, stream=None):
    """attention_rel_pos over heads x windows straight from a window-major
    qkv projection [windows * h * w, 3 * heads * hd] into the merged rows out
    [windows * h * w, heads * hd] (new; a bfloat16 out: the output rounded to
    bf16 in the epilogue)."""
    width, n = heads * hd, h * w
    base = _ptr(qkv)
    bf16 = out.dtype == _torch().bfloat16
    name = "uocr_rocm_attention_rel_pos_windows_bf16_ws" if bf16 else "uocr_rocm_attention_rel_pos_windows_ws"
    _op(name, stream, base, 3 * width, hd, n * 3 * width, base + 4 * width,
        3 * width, hd, n * 3 * width, base + 8 * width, 3 * width, hd, n * 3 * width, _ptr(out), width, hd, n * width,
        heads, windows, h, w, hd, scale, _ptr(rh), _ptr(rw), _ptr(workspace), workspace.numel())


def attention_rel_pos_workspace_floats(slices, h, w):
    """Floats of the workspace attention_rel_pos forms the bias's dots in."""
    return int(lib().uocr_rocm_attention_rel_pos_workspace_floats(slices, h, w))


def split_heads(x, parts, heads, hd, y, stream=None):
    """y [parts, heads, rows, hd] = x [rows, parts * heads * hd] (new)."""
    _op("uocr_rocm_split_heads", stream, _ptr(x), x.shape[0], parts, heads, hd, _ptr(y))


def merge_heads(x, y, stream=None):
    """y [rows, heads * hd] = x [heads, rows, hd] (new)."""
    heads, rows, hd = x.shape
    _op("uocr_rocm_merge_heads", stream, _ptr(x), heads, rows, hd, _ptr(y))


def rel_pos_bias(q, ldq, h, w, d, rh, rw, bias, q_offset=0, stream=None):
    """bias [h w, h w] of one window and head; the query rows start q_offset
    floats into q (a head's columns). Reference: rel_pos_bias, ops.h:91-95."""
    _op("uocr_rocm_rel_pos_bias", stream, _ptr(q) + 4 * q_offset, ldq, h, w, d, _ptr(rh), _ptr(rw), _ptr(bias))


def rel_pos_softmax_rows(scores, windows, q, ldq, h, w, d, rh, rw, q_offset=0, stream=None):
    """scores [windows, h w, h w] = softmax(scores + rel_pos_bias) per row,
    query rows from q_offset floats into q (new)."""
    _op("uocr_rocm_rel_pos_softmax_rows", stream, _ptr(scores), windows, _ptr(q) + 4 * q_offset, ldq, h, w, d,
        _ptr(rh), _ptr(rw))


def append_step(cache, row, state, capacity=None, stream=None):
    """cache[state.pos] = row for a cache [capacity, width] (float32).
    Reference: append_step, decode_ops.h:28-29."""
    width = row.numel()
    cap = cache.numel() // width if capacity is None and width else (-1 if capacity is None else capacity)
    name = "uocr_rocm_append_step_bf16" if _is_bf16(cache) else "uocr_rocm_append_step"
    _op(name, stream, _ptr(cache), _ptr(row), width, _ptr(state), cap)


def attend_scratch_floats(heads, hd, capacity) -> int:
    """Floats of scratch that attend_step needs. Reference: decode_ops.h:42-43."""
    return int(lib().uocr_rocm_attend_scratch_floats(heads, hd, capacity))


def attend_step(q, k_cache, v_cache, heads, hd, mask, scale, state, scratch, out, stream=None):
    """Masked attention of the one query q [heads * hd] over the keys
    0..state.pos of k_cache / v_cache [capacity, heads * hd] (float32).
    Reference: attend_step, decode_ops.h:44-47."""
    capacity = k_cache.numel() // (heads * hd) if heads * hd else 0
    if v_cache.numel() != k_cache.numel() or q.numel() != heads * hd or out.numel() != heads * hd:
        raise ValueError("attend_step shapes: q, out [heads * hd]; k_cache, v_cache [capacity, heads * hd]")
    if mask is not None and mask.numel() < capacity:
        raise ValueError("mask must hold capacity floats")
    if scratch.numel() < attend_scratch_floats(heads, hd, capacity):
        raise ValueError("scratch is smaller than attend_scratch_floats(heads, hd, capacity)")
    bf = _is_bf16(k_cache)
    if _is_bf16(v_cache) != bf:
        raise ValueError("k_cache and v_cache must share a dtype")
    _op("uocr_rocm_attend_step_bf16" if bf else "uocr_rocm_attend_step", stream, _ptr(q), _ptr(k_cache),
        _ptr(v_cache), heads, hd, _f32_param(mask), scale, _ptr(state), _ptr(scratch), capacity, _ptr(out))


def attend_step_noalloc(q, k_cache, v_cache, heads, hd, mask, scale, state, out, stream=None):
    """attend_step with no scratch argument: the split records go to the
    library's fixed per-device array (at most 1,048,576 floats), so the call
    allocates nothing. Calls that overlap on one GPU race on that array."""
    capacity = k_cache.numel() // (heads * hd) if heads * hd else 0
    if v_cache.numel() != k_cache.numel() or q.numel() != heads * hd or out.numel() != heads * hd:
        raise ValueError("attend_step_noalloc shapes: q, out [heads * hd]; k_cache, v_cache [capacity, heads * hd]")
    if mask is not None and mask.numel() < capacity:
        raise ValueError("mask must hold capacity floats")
    if _is_bf16(k_cache) or _is_bf16(v_cache):
        raise ValueError("attend_step_noalloc takes float32 caches")
    _op("uocr_rocm_attend_step_noalloc", stream, _ptr(q), _ptr(k_cache), _ptr(v_cache), heads, hd,
        _f32_param(mask), scale, _ptr(state), capacity, _ptr(out))


# ---- the block router (src/backend/cuda/ops.h:97-124, decode_ops.h:30-40) --------------------


def _i64_param(t):
    torch = _torch()
    if t is not None and t.dtype != torch.int64:
        raise ValueError("block pages and query pages are int64")
    return _ptr(t)


def block_summaries(keys, head_cls, block_size, out, stream=None):
    """out [ceil(s / block_size), d]: per block of router keys [s, d], the
    softmax(clamp(k . head_cls / sqrt d))-weighted mean of its keys."""
    s, d = _rows_cols(keys)
    if out.numel() != ((s + block_size - 1) // block_size) * d or head_cls.numel() != d:
        raise ValueError("block_summaries shapes: keys [s, d], head_cls [d], out [ceil(s / block_size), d]")
    _op("uocr_rocm_block_summaries", stream, _f32_param(keys), s, d, _f32_param(head_cls), block_size, _ptr(out))


def summary_step(router_keys, d, head_cls, block_size, state, summaries, stream=None):
    """The summary of the block holding state.pos, into summaries [max_blocks, d]."""
    max_blocks = summaries.numel() // d
    _op("uocr_rocm_summary_step", stream, _f32_param(router_keys), d, _f32_param(head_cls), block_size, _ptr(state),
        max_blocks, _ptr(summaries))


def scores_step(rq, summaries, d, block_size, state, z, stream=None):
    """z[b] = rq . summaries[b] / sqrt d up to the block holding state.pos (z [max_blocks])."""
    _op("uocr_rocm_scores_step", stream, _f32_param(rq), _f32_param(summaries), d, block_size, _ptr(state),
        z.numel(), _ptr(z))


def route_blocks(z, first_pos, keys, block_min, block_max, query_page, one_page, params, mask, stream=None):
    """Key masks [rows, keys] of prompt rows from scores z [rows, nblk]."""
    rows, nblk = _rows_cols(z)
    if mask.numel() != rows * keys:
        raise ValueError("route_blocks: mask [rows, keys]")
    pb = 0 if block_min is None else block_min.numel()
    _op("uocr_rocm_route_blocks", stream, _f32_param(z), rows, nblk, first_pos, keys, _i64_param(block_min),
        _i64_param(block_max), pb, _i64_param(query_page), one_page, ctypes.byref(params), _ptr(mask))


def route_step(z, block_min, block_max, state, params, mask, stream=None):
    """The key mask mask[0..pos] of the decode query at state.pos from z [max_blocks]."""
    pb = 0 if block_min is None else block_min.numel()
    _op("uocr_rocm_route_step", stream, _f32_param(z), z.numel(), _i64_param(block_min), _i64_param(block_max), pb,
        _ptr(state), ctypes.byref(params), _ptr(mask))


MAX_KEY_SEGMENTS = 33  # UOCR_ROCM_MAX_KEY_SEGMENTS
KEY_SEGMENT_WORDS = 4 * (1 + MAX_KEY_SEGMENTS)


def route_decode_step(rq, rk, q_norm, k_norm, eps, inv_tok, inv_page, page_mod, head_cls, router_keys, summaries,
                      block_min, block_max, state, params, mask, z_out=None, rqk_out=None, segments=None,
                      stream=None):
    """The router half of a decode step in one launch: router norms, rope,
    the router key's append, the block summary, the scores and the route into
    mask [capacity] (keys 0..pos). router_keys [capacity, d]. segments (int32
    [KEY_SEGMENT_WORDS] or None) receives the keys the mask keeps: the count,
    the live keys, then {first key, keys, bias bits, 0} per segment; with
    segments, mask may be None (not written)."""
    d = rq.numel()
    capacity = router_keys.numel() // d
    n_tok = 0 if inv_tok is None else inv_tok.numel()
    pb = 0 if block_min is None else block_min.numel()
    if (mask is None and segments is None) or (mask is not None and mask.numel() < capacity):
        raise ValueError("route_decode_step: mask [capacity] (or None with segments)")
    if segments is not None and (segments.dtype != _torch().int32 or segments.numel() < KEY_SEGMENT_WORDS):
        raise ValueError("route_decode_step: segments int32 [KEY_SEGMENT_WORDS]")
    _op("uocr_rocm_route_decode_step_segments", stream, _f32_param(rq), _f32_param(rk), _f32_param(q_norm),
        _f32_param(k_norm), eps, _f32_param(inv_tok), n_tok, _f32_param(inv_page), page_mod, _f32_param(head_cls),
        _ptr(router_keys), _ptr(summaries), d, _i64_param(block_min), _i64_param(block_max), pb, _ptr(state),
        ctypes.byref(params), capacity, _ptr(mask), _ptr(z_out), _ptr(rqk_out), _ptr(segments))


# ---- fused decode-step ops -------------------------------------------------------------------


def embed_add_rms_norm_step(table, state, w, x, h, delta=None, eps=1e-6, stream=None):
    """x = table[state.token] (+ delta); h = rms_norm(x) * w, in one launch
    (x, h float32 or bfloat16 alike; delta the same dtype or None)."""
    bf = _is_bf16(x)
    if _is_bf16(h) != bf or (delta is not None and _is_bf16(delta) != bf):
        raise ValueError("x, h and delta must share a dtype")
    cols = table.shape[-1]
    if x.numel() != cols or h.numel() != cols or (delta is not None and delta.numel() != cols):
        raise ValueError("x, h and delta must hold one table row")
    name = "uocr_rocm_embed_add_rms_norm_step_bf16" if bf else "uocr_rocm_embed_add_rms_norm_step"
    _op(name, stream, _ptr(table), table.shape[0], _ptr(state), _ptr(delta), _f32_param(w), _ptr(x), _ptr(h), cols,
        eps)


def add_rms_norm_gemv_bf16(x, w, y, delta=None, x_out=None, w_norm=None, eps=1e-6, h_out=None, bias=None,
                           stream=None):
    """y = bf16(h) . w^T (+ bias) with h = rms_norm(x + delta) * w_norm in one
    launch; x_out receives x + delta and h_out the fp32 h when given."""
    n, k = w.shape
    _op("uocr_rocm_add_rms_norm_gemv_bf16", stream, _ptr(x), _ptr(delta), _ptr(x_out), _f32_param(w_norm), eps,
        _ptr(h_out), k, _ptr(w), n, _f32_param(bias), _ptr(y))


def add_rms_norm_swiglu_gemv_bf16(x, w_gate, w_up, act, delta=None, x_out=None, w_norm=None, eps=1e-6, h_out=None,
                                  stream=None):
    """act = silu(bf16(h) . w_gate^T) * (bf16(h) . w_up^T), h as above, in one launch."""
    ffn, k = w_gate.shape
    if tuple(w_up.shape) != (ffn, k):
        raise ValueError("w_gate and w_up must have the same shape")
    _op("uocr_rocm_add_rms_norm_swiglu_gemv_bf16", stream, _ptr(x), _ptr(delta), _ptr(x_out), _f32_param(w_norm),
        eps, _ptr(h_out), k, _ptr(w_gate), _ptr(w_up), ffn, _ptr(act))


def add_rms_norm_swiglu_router_gemv_bf16(x, w_gate, w_up, act, router, logits, delta=None, x_out=None, w_norm=None,
                                         eps=1e-6, h_out=None, stream=None):
    """add_rms_norm_swiglu_gemv_bf16 and, in the same launch, logits =
    router (fp32 [experts, k]) . h with h unrounded."""
    ffn, k = w_gate.shape
    experts = router.shape[0]
    if tuple(w_up.shape) != (ffn, k) or tuple(router.shape) != (experts, k) or logits.numel() != experts:
        raise ValueError("w_gate, w_up [ffn, k]; router [experts, k]; logits [experts]")
    if router.dtype != _torch().float32 or logits.dtype != _torch().float32:
        raise ValueError("router and logits must be float32")
    _op("uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16", stream, _ptr(x), _ptr(delta), _ptr(x_out),
        _f32_param(w_norm), eps, _ptr(h_out), k, _ptr(w_gate), _ptr(w_up), ffn, _ptr(act), _ptr(router), experts,
        _ptr(logits))


def attend_rope_kv_step(q, k_row, v_row, k_cache, v_cache, heads, hd, mask, scale, state, inv_tok, inv_page,
                        page_mod, scratch, out, stream=None):
    """rope_qk_step on (q, k_row), append of the rotated key and v_row at
    state.pos, and attend_step, in two launches (q, k_row, v_row untouched)."""
    capacity = k_cache.numel() // (heads * hd) if heads * hd else 0
    if scratch.numel() < attend_scratch_floats(heads, hd, capacity):
        raise ValueError("scratch is smaller than attend_scratch_floats(heads, hd, capacity)")
    n_tok = 0 if inv_tok is None else inv_tok.numel()
    bf = _is_bf16(k_cache)
    if _is_bf16(v_cache) != bf:
        raise ValueError("k_cache and v_cache must share a dtype")
    name = "uocr_rocm_attend_rope_kv_step_bf16" if bf else "uocr_rocm_attend_rope_kv_step"
    _op(name, stream, _ptr(q), _ptr(k_row), _ptr(v_row), _ptr(k_cache), _ptr(v_cache),
        heads, hd, _f32_param(mask), scale, _ptr(state), _f32_param(inv_tok), n_tok, _f32_param(inv_page), page_mod,
        _ptr(scratch), capacity, _ptr(out))


def attend_segments_scratch_floats(heads, hd, max_live):
    """Scratch floats of attend_rope_kv_step_segments."""
    return int(lib().uocr_rocm_attend_segments_scratch_floats(heads, hd, max_live))


def attend_rope_kv_step_segments(q, k_row, v_row, k_cache, v_cache, heads, hd, segments, max_live, scale, state,
                                 inv_tok, inv_page, page_mod, scratch, out, stream=None):
    """attend_rope_kv_step over the live keys that route_decode_step listed in
    segments (int32) instead of a mask; max_live bounds their count and fixes
    the split count. out None: the split records stay in scratch for
    attend_merge_gemv_bf16."""
    capacity = k_cache.numel() // (heads * hd) if heads * hd else 0
    if segments.dtype != _torch().int32 or segments.numel() < KEY_SEGMENT_WORDS:
        raise ValueError("segments must be int32 [KEY_SEGMENT_WORDS]")
    if scratch.numel() < attend_segments_scratch_floats(heads, hd, max_live):
        raise ValueError("scratch is smaller than attend_segments_scratch_floats(heads, hd, max_live)")
    n_tok = 0 if inv_tok is None else inv_tok.numel()
    bf = _is_bf16(k_cache)
    if _is_bf16(v_cache) != bf:
        raise ValueError("k_cache and v_cache must share a dtype")
    name = "uocr_rocm_attend_rope_kv_step_segments_bf16" if bf else "uocr_rocm_attend_rope_kv_step_segments"
    _op(name, stream, _ptr(q), _ptr(k_row), _ptr(v_row), _ptr(k_cache), _ptr(v_cache), heads, hd, _ptr(segments),
        max_live, scale, _ptr(state), _f32_param(inv_tok), n_tok, _f32_param(inv_page), page_mod, _ptr(scratch),
        capacity, _ptr(out))


def attend_merge_gemv_bf16(scratch, heads, hd, max_live, w, y, bias=None, x_out=None, stream=None):
    """y = bf16(merge) . w^T (+ bias) where merge is the attention row that
    attend_rope_kv_step_segments (out=None, the same heads, hd, max_live) left
    as split records in scratch; x_out receives the merged row."""
    n, k = w.shape
    if k != heads * hd or y.numel() != n or (x_out is not None and x_out.numel() != k):
        raise ValueError("w [n, heads * hd], y [n], x_out [heads * hd]")
    if scratch.numel() < attend_segments_scratch_floats(heads, hd, max_live):
        raise ValueError("scratch is smaller than attend_segments_scratch_floats(heads, hd, max_live)")
    _op("uocr_rocm_attend_merge_gemv_bf16", stream, _ptr(scratch), heads, hd, max_live, _ptr(w), n,
        _f32_param(bias), _ptr(y), _ptr(x_out))


# ---- mixture of experts at decode -------------------------------------------------------------


def expert_topk(logits, k, ids, weights, stream=None):
    """Softmax over each row of logits [rows, experts] (float32), then the top
    k (lower index on a tie): ids [rows, k] int64, weights [rows, k] float32.
    Reference: expert_topk, src/backend/cuda/ops.h:77-81."""
    rows, experts = _rows_cols(logits)
    if logits.dtype != _torch().float32 or ids.numel() != rows * k or weights.numel() != rows * k:
        raise ValueError("expert_topk: float32 logits [rows, experts], ids and weights [rows, k]")
    _op("uocr_rocm_expert_topk", stream, _ptr(logits), rows, experts, k, _ptr(ids), _ptr(weights))


def expert_scratch_floats(k: int, ffn: int) -> int:
    """Floats of scratch that expert_ffn_one needs."""
    return int(lib().uocr_rocm_expert_scratch_floats(k, ffn))


def gemv_f32(x, w, y, bias=None, stream=None):
    """y = x . w^T (+ bias) with float32 weights w [n, k], x not rounded: the
    gate logits (src/model/cuda/cuda_decoder.cpp:141-142)."""
    n, k = w.shape
    if w.dtype != _torch().float32 or x.numel() != k or y.numel() != n:
        raise ValueError("gemv_f32: float32 w [n, k], x [k], y [n]")
    _op("uocr_rocm_gemv_f32", stream, _ptr(x), k, _ptr(w), n, _f32_param(bias), _ptr(y))


def expert_ffn_one(x, gate, up, down, ids, weights, scratch, out, base=None, stream=None):
    """One decode row x [hidden] through its k routed experts: gate/up
    [experts, ffn, hidden] (or [experts * ffn, hidden]) and down [experts,
    hidden, ffn] bf16 stacks, ids [k] int64, weights [k] float32.
    Reference: expert_ffn_one, src/backend/cuda/ops.h:82-90."""
    hidden = x.numel()
    ffn = down.shape[-1]
    experts = down.numel() // (hidden * ffn) if hidden * ffn else 0
    k = ids.numel()
    if gate.numel() != experts * ffn * hidden or up.numel() != gate.numel() or out.numel() != hidden:
        raise ValueError("expert_ffn_one shapes: gate/up [experts, ffn, hidden], down [experts, hidden, ffn]")
    if weights.numel() != k or scratch.numel() < expert_scratch_floats(k, ffn):
        raise ValueError("expert_ffn_one: weights [k] and scratch of expert_scratch_floats(k, ffn) floats")
    if base is not None and base.numel() != hidden:
        raise ValueError("expert_ffn_one: base [hidden]")
    _op("uocr_rocm_expert_ffn_one", stream, _ptr(x), hidden, ffn, _ptr(gate), _ptr(up), _ptr(down), experts,
        _ptr(ids), _ptr(weights), k, _ptr(base), _ptr(scratch), _ptr(out))


def moe_ffn_one(x, gate, up, down, logits, ids, weights, shared_act, shared_down, scratch, out, stream=None):
    """The routed experts from the router's logits [experts] (their top k
    written to ids [k] and weights [k]) plus the shared experts' down product
    in the same launch: out = bf16(shared_act) . shared_down^T + the routed
    sum (shared_down [hidden, shared_ffn] bf16)."""
    hidden = x.numel()
    ffn = down.shape[-1]
    experts = down.numel() // (hidden * ffn) if hidden * ffn else 0
    k = ids.numel()
    shared_ffn = shared_down.shape[-1]
    if gate.numel() != experts * ffn * hidden or up.numel() != gate.numel() or out.numel() != hidden:
        raise ValueError("moe_ffn_one shapes: gate/up [experts, ffn, hidden], down [experts, hidden, ffn]")
    if logits.numel() != experts or logits.dtype != _torch().float32:
        raise ValueError("moe_ffn_one: float32 logits [experts]")
    if shared_down.numel() != hidden * shared_ffn or shared_act.numel() != shared_ffn:
        raise ValueError("moe_ffn_one: shared_down [hidden, shared_ffn], shared_act [shared_ffn]")
    if weights.numel() != k or scratch.numel() < expert_scratch_floats(k, ffn):
        raise ValueError("moe_ffn_one: weights [k] and scratch of expert_scratch_floats(k, ffn) floats")
    _op("uocr_rocm_moe_ffn_one", stream, _ptr(x), hidden, ffn, _ptr(gate), _ptr(up), _ptr(down), experts,
        _ptr(logits), k, _ptr(ids), _ptr(weights), _ptr(shared_act), _ptr(shared_down), shared_ffn, _ptr(scratch),
        _ptr(out))
