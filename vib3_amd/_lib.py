"""ctypes binding of libvib3_hip.so (the C ABI declared in include/vib3_hip.h).

The library is built in-tree by vib3_amd/build.py. There is no fallback: if the shared object is
missing or fails to load, every entry point raises, so a GPU run can never silently compute on
the CPU.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# VIB3_LIB may point at another build of the same ABI (e.g. an instrumented one)
LIB_PATH = os.environ.get("VIB3_LIB") or os.path.join(HERE, "libvib3_hip.so")

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
ROUTER_SOFTMAX, ROUTER_SIGMOID = 0, 1
MOE_F32_INTERMEDIATE = 1
MOE_TEST_ROUTER_TIMEOUT = 0x100
MOE_SEPARATE_PROLOGUE = 0x200

ERRORS = {-1: "unsupported shape or dtype", -2: "bad count", -3: "bad pointer or alignment",
          -4: "workspace too small", -5: "unexpected .vib3 file or page layout",
          -6: ".vib3 file cannot be opened", -7: "a page is not resident"}


class Vib3Error(RuntimeError):
    """A launcher returned non-zero (hipError_t > 0, argument error < 0)."""

    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} failed: {ERRORS.get(code, f'hipError_t {code}')} (code {code})")
        self.code = code


class MoeInt4Layer(C.Structure):
    """vib3_moe_int4_layer (include/vib3_hip.h)."""

    _fields_ = [
        ("x", C.c_void_p), ("x_dtype", C.c_int), ("hidden", C.c_int), ("inter", C.c_int),
        ("group_size", C.c_int), ("scale_dtype", C.c_int),
        ("router_w", C.c_void_p), ("router_w_dtype", C.c_int), ("router_bias", C.c_void_p),
        ("num_experts", C.c_int), ("top_k", C.c_int), ("scoring_mode", C.c_int),
        ("scaling_factor", C.c_float), ("normalize", C.c_int),
        ("in_ids", C.c_void_p), ("in_weights", C.c_void_p),
        ("page_table", C.c_void_p), ("shared_page_table", C.c_void_p), ("num_shared", C.c_int),
        ("max_pages", C.c_int), ("rows_per_page", C.c_int * 3), ("flags", C.c_int),
        ("out", C.c_void_p), ("out_ids", C.c_void_p), ("out_weights", C.c_void_p),
        ("out_scores", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("norm_weight", C.c_void_p), ("norm_eps", C.c_float), ("residual", C.c_void_p),
        ("shared_gate", C.c_void_p),
    ]


class ResolvedPage(C.Structure):
    """vib3_resolved_page (include/vib3_hip.h): query_planner.rs:38-43 ResolvedPage."""

    _fields_ = [
        ("layer", C.c_uint16), ("expert", C.c_uint16), ("segment", C.c_uint16),
        ("page_idx", C.c_uint16), ("device_ptr", C.c_uint64), ("row_start", C.c_uint16),
        ("row_count", C.c_uint16),
    ]


class MoeMxfp4Batch(C.Structure):
    """vib3_moe_mxfp4_batch (include/vib3_hip.h)."""

    _fields_ = [
        ("x", C.c_void_p), ("tokens", C.c_int), ("hidden", C.c_int), ("inter", C.c_int),
        ("num_experts", C.c_int), ("top_k", C.c_int), ("ids", C.c_void_p),
        ("weights", C.c_void_p), ("page_table", C.c_void_p), ("out", C.c_void_p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


# name -> (restype, argtypes); every symbol declared in include/vib3_hip.h
P, I, F, S, U64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint64
SIGNATURES = {
    "vib3_launch_partial_matmul_int4": (I, [P, P, P, P, I, I, I, P]),
    "vib3_launch_partial_matmul_int4_f32": (I, [P, P, P, P, I, I, I, P]),
    "vib3_launch_fused_swiglu_int4_f32": (I, [P, P, P, P, P, P, I, I, I, P]),
    "vib3_launch_silu_mul": (I, [P, P, P, I, P]),
    "vib3_launch_weighted_accumulate_f32": (I, [P, P, F, I, P]),
    "vib3_launch_weighted_accumulate_f32_f32": (I, [P, P, F, I, P]),
    "vib3_launch_weighted_accumulate": (I, [P, P, F, I, P]),
    "vib3_launch_weighted_accumulate_f32_dev_scalar": (I, [P, P, P, I, P]),
    "vib3_launch_router_gemv": (I, [P, P, P, I, I, P]),
    "vib3_launch_router_gemv_f32": (I, [P, P, P, I, I, P]),
    "vib3_launch_router_topk": (I, [P, P, P, P, P, P, I, I, I, I, F, P]),
    "vib3_launch_rms_norm_f32": (I, [P, P, P, I, F, P]),
    "vib3_launch_rms_norm_f32_to_f16": (I, [P, P, P, I, F, P]),
    "vib3_launch_residual_add_f32_f32": (I, [P, P, I, P]),
    "vib3_launch_sigmoid_gated_accumulate_f32": (I, [P, P, P, I, P]),
    "vib3_launch_partial_matmul_int4_ex": (I, [P, I, P, P, I, I, I, I, I, P]),
    "vib3_launch_partial_swiglu_int4_ex": (I, [P, I, P, P, P, I, I, I, I, I, P]),
    "vib3_router_workspace_bytes": (S, [I]),
    "vib3_launch_router_topk_ex": (I, [P, I, P, I, P, I, I, I, I, F, I, P, P, P, P, P]),
    "vib3_moe_int4_workspace_bytes": (S, [C.POINTER(MoeInt4Layer)]),
    "vib3_launch_moe_int4_layer": (I, [C.POINTER(MoeInt4Layer), P]),
    "vib3_moe_int4_router_fused": (I, [C.POINTER(MoeInt4Layer)]),
    "vib3_moe_int4_layer_status": (I, [C.POINTER(MoeInt4Layer), I, P]),
    "vib3_launch_moe_int4_layer_noalloc": (I, [C.POINTER(MoeInt4Layer), P]),
    "vib3_launch_moe_int4_layer_stage": (I, [C.POINTER(MoeInt4Layer), I, P]),
    "vib3_moe_mxfp4_workspace_bytes": (S, [C.POINTER(MoeMxfp4Batch)]),
    "vib3_launch_moe_mxfp4_batched": (I, [C.POINTER(MoeMxfp4Batch), P]),
    "vib3_hip_zero": (I, [P, S, P]),
    "vib3_synth_bytes": (I, [P, S, U64, U64, S, P]),
    "vib3_synth_normal": (I, [P, I, S, U64, U64, S, F, P]),
    "vib3_synth_int4_page": (I, [P, U64, U64, I, I, I, F, I, I, P]),
    "vib3_synth_mxfp4_page": (I, [P, U64, U64, I, I, I, P]),
    "vib3_file_open": (I, [C.c_char_p, P]),
    "vib3_file_close": (None, [P]),
    "vib3_file_get_info": (I, [P, P]),
    "vib3_file_metadata": (I, [P, P, P]),
    "vib3_file_page": (I, [P, C.c_uint32, P]),
    "vib3_file_expert_pages": (I, [P, C.c_uint16, C.c_uint16, P, I, P]),
    "vib3_file_page_data": (I, [P, C.c_uint32, P, P]),
    "vib3_file_read_page": (I, [P, C.c_uint32, P, S, P]),
    "vib3_build_page_table": (I, [P, C.c_uint16, P, I, P, P, P, I, P, P]),
    "vib3_build_page_table_resolved": (I, [P, S, P, I, P, P, P, I, P, P, I, P]),
    "vib3_launch_quantize_activation_fp4": (I, [P, P, P, I, P]),
    "vib3_launch_fused_rms_norm_quantize_fp4": (I, [P, P, P, P, P, I, F, P]),
    "vib3_launch_quantize_activation_fp4_fast": (I, [P, P, P, I, P]),
    "vib3_moe_prewarm_gpu_bufs": (I, [I, I]),
    "vib3_launch_moe_experts_fused": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, P, P]),
    "vib3_launch_moe_experts_fused_gpu": (I, [P, P, P, P, P, I, I, I, I, I, I, I, P, P]),
    "vib3_launch_repack_weights_inplace": (I, [P, C.c_longlong, P]),
    "vib3_launch_repack_row_to_tiled": (I, [P, P, I, I, P]),
    "vib3_hip_version": (C.c_char_p, []),
    "vib3_moe_experts_fused_workspace_bytes": (S, [I]),
    "vib3_launch_moe_experts_fused_ws": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, P, P, S, P]),
    "vib3_launch_moe_experts_fused_gpu_ws": (I, [P, P, P, P, P, I, I, I, I, I, I, I, P, P, S, P]),
    "vib3_launch_expert_batched": (I, [P, P, P, P, P, P, P, P, P, F, I, I, I, I, P]),
    "vib3_launch_fp16_to_nvfp4_weight": (I, [P, P, P, I, I, P]),
    "vib3_launch_gemv_mma_nvfp4_preq": (I, [P, P, P, P, P, I, I, P]),
    "vib3_launch_gemv_mma_nvfp4_preq_fast": (I, [P, P, P, P, P, I, I, P]),
    "vib3_launch_fused_swiglu_mma_nvfp4_preq": (I, [P, P, P, P, P, P, P, I, I, P]),
    "vib3_launch_fused_swiglu_mma_nvfp4_preq_fast": (I, [P, P, P, P, P, P, P, I, I, P]),
    "vib3_launch_gemv_mma_nvfp4_tiled": (I, [P, P, P, P, P, I, I, P]),
    "vib3_launch_gemv_scalar_nvfp4": (I, [P, P, P, P, P, I, I, P]),
    "vib3_launch_gemv_mma_nvfp4": (I, [P, P, P, P, I, I, P]),
    "vib3_launch_fused_swiglu_mma_nvfp4": (I, [P, P, P, P, P, P, I, I, P]),
    "vib3_launch_partial_matmul_nvfp4": (I, [P, P, P, P, I, I, I, P]),
    "vib3_launch_partial_matmul_nvfp4_f32out": (I, [P, P, P, P, I, I, I, P]),
    "vib3_launch_partial_matmul_nvfp4_fp16in": (I, [P, P, P, P, I, I, I, P]),
    "vib3_launch_fused_swiglu_nvfp4": (I, [P, P, P, P, P, P, I, I, I, P]),
    "vib3_launch_fused_swiglu_nvfp4_f32out": (I, [P, P, P, P, P, P, I, I, I, P]),
}

_lib = None


def load() -> C.CDLL:
    """Load libvib3_hip.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
                " or `python vib3_amd/build.py`")
        lib = C.CDLL(LIB_PATH)
        alt = bool(os.environ.get("VIB3_LIB"))  # another build may predate some entry points
        for name, (res, args) in SIGNATURES.items():
            if alt and not hasattr(lib, name):
                continue
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call a launcher and raise Vib3Error on a non-zero return."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise Vib3Error(name, rc)
