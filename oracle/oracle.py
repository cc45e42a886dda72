"""ctypes front end of the CPU oracle (oracle/cpu_ref.c). TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
module, and only to check or to time the reference algorithm. Each function names the
reference code it restates (threehundobaud/vic, crate ``vib3``).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, BF16 = 0, 1, 2
_lib = None


def build() -> None:
    """Compile liboracle.so from cpu_ref.c (gcc, -ffp-contract=off)."""
    subprocess.check_call(["make", "-s", "-B", "-C", _HERE, "all"])


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L: C.CDLL) -> None:
    P, S, I, F, U64 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint64
    sig = {
        "v3o_f32_to_f16": (C.c_uint16, [F]),
        "v3o_f16_to_f32": (F, [C.c_uint16]),
        "v3o_f32_to_bf16": (C.c_uint16, [F]),
        "v3o_bf16_to_f32": (F, [C.c_uint16]),
        "v3o_default_threads": (I, []),
        "v3o_matmul_int4_acc": (None, [P, P, S, S, S, I, P, I]),
        "v3o_partial_matmul_int4": (None, [P, P, P, S, S]),
        "v3o_swiglu_int4_acc": (None, [P, P, P, S, S, S, I, P, I]),
        "v3o_partial_swiglu_int4": (None, [P, P, P, P, S, S]),
        "v3o_weighted_accumulate_f32": (None, [P, P, F, S]),
        "v3o_weighted_accumulate_f16": (None, [P, P, F, S]),
        "v3o_fp4_e8m0_of_amax": (C.c_uint8, [F]),
        "v3o_e2m1_rne": (C.c_uint8, [F]),
        "v3o_exp_cw": (F, [F]),
        "v3o_fp4_quantize_act": (None, [P, S, P, P]),
        "v3o_fp4_norm_inv": (F, [P, S, F]),
        "v3o_fused_rms_norm_quantize_fp4": (None, [P, P, S, F, P, P, P]),
        "v3o_nvfp4_matvec": (None, [P, P, P, P, S, S, P]),
        "v3o_moe_experts_fused": (None, [P, P, P, P, P, S, S, S, S, P]),
        "v3o_fp4_split_half": (None, [P, S]),
        "v3o_fp4_to_tiled": (None, [P, P, S, S]),
        "v3o_router": (I, [P, P, I, S, S, S, I, F, I, P, P, P, P, I]),
        "v3o_quantize_int4": (None, [P, S, S, S, P]),
        "v3o_dequantize_int4": (None, [P, S, S, S, I, P]),
        "v3o_moe_layer": (None, [P, S, S, S, I, P, P, P, S, P, S, I, P, I]),
        "v3o_moe_layer_w": (None, [P, S, S, S, I, P, P, P, S, P, S, P, I, P, I]),
        "v3o_inv_rms": (F, [P, S, F]),
        "v3o_rms_norm_f32": (None, [P, S, P, F, P]),
        "v3o_residual_add_f32": (None, [P, P, S]),
        "v3o_linear_row_f16": (F, [P, P, S]),
        "v3o_sigmoid": (F, [F]),
        "v3o_e2m1": (F, [C.c_uint8]),
        "v3o_e8m0": (F, [C.c_uint8]),
        "v3o_matmul_mxfp4_acc": (None, [P, P, P, S, S, P, I]),
        "v3o_synth_hash": (U64, [U64, U64, U64]),
        "v3o_synth_normal": (F, [U64, U64, U64]),
        "v3o_synth_bytes": (None, [U64, U64, S, S, P]),
        "v3o_synth_scale": (C.c_uint16, [U64, U64, U64, F, I]),
        "v3o_synth_normal_array": (None, [U64, U64, S, S, F, I, P]),
        "v3o_synth_int4_page": (None, [U64, U64, S, S, I, F, S, S, P]),
        "v3o_moe_mxfp4_batched": (None, [P, S, S, S, P, S, P, P, S, P, I]),
        "v3o_synth_e8m0": (C.c_uint8, [U64, U64, U64]),
        "v3o_synth_mxfp4_page": (None, [U64, U64, S, S, S, P]),
        "v3o_nvfp4_page_bytes": (S, [S, S]),
        "v3o_quantize_weights_to_nvfp4": (None, [P, S, S, P]),
        "v3o_quantize_half_to_nvfp4": (None, [P, I, S, S, P]),
        "v3o_convert_int4_to_nvfp4": (None, [P, S, S, S, S, P]),
        "v3o_fp16_to_nvfp4_weight": (None, [P, S, S, P, P]),
        "v3o_nvfp4_seq_matvec_f64": (None, [P, P, P, S, S, P]),
        "v3o_nvfp4_page_matvec": (None, [P, P, P, P, S, S, I, I, P]),
        "v3o_nvfp4_page_swiglu": (None, [P, P, P, P, P, P, S, S, I, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- conversions

def f16_bits(x) -> np.ndarray:
    """f32 -> f16 bit patterns (RNE), via the oracle's own converter."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    fn = lib().v3o_f32_to_f16
    return np.array([fn(float(v)) for v in x], dtype=np.uint16)


def to_f32(bits: np.ndarray, dt: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits)
    if dt == F32:
        return bits.astype(np.float32)
    if dt == BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- kernels

def matmul_int4_acc(x: np.ndarray, page: np.ndarray, k: int, m: int, g: int, scale_dt: int,
                    nthreads: int = 0) -> np.ndarray:
    """kernels.rs:2746 cpu_matmul_int4_grouped, fp32 accumulators before f16 rounding."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    page = np.ascontiguousarray(page, dtype=np.uint8)
    out = np.empty(m, dtype=np.float32)
    lib().v3o_matmul_int4_acc(_p(x), _p(page), k, m, g, scale_dt, _p(out), nthreads)
    return out


def partial_matmul_int4(x_f16: np.ndarray, page: np.ndarray, k: int, m: int) -> np.ndarray:
    """kernels.rs:25 partial_matmul(DType::INT4) CPU branch: f16 bits in and out."""
    x_f16 = np.ascontiguousarray(x_f16, dtype=np.uint16)
    page = np.ascontiguousarray(page, dtype=np.uint8)
    out = np.empty(m, dtype=np.uint16)
    lib().v3o_partial_matmul_int4(_p(x_f16), _p(page), _p(out), k, m)
    return out


def swiglu_int4_acc(x, up_page, gate_page, k, m, g, scale_dt, nthreads=0) -> np.ndarray:
    """kernels.rs:2932 cpu_swiglu_int4, silu(gate)*up in fp32 before f16 rounding."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    up_page = np.ascontiguousarray(up_page, dtype=np.uint8)
    gate_page = np.ascontiguousarray(gate_page, dtype=np.uint8)
    out = np.empty(m, dtype=np.float32)
    lib().v3o_swiglu_int4_acc(_p(x), _p(up_page), _p(gate_page), k, m, g, scale_dt, _p(out), nthreads)
    return out


def partial_swiglu_int4(x_f16, up_page, gate_page, k, m) -> np.ndarray:
    """kernels.rs:162 partial_swiglu(DType::INT4) CPU branch: f16 bits in and out."""
    x_f16 = np.ascontiguousarray(x_f16, dtype=np.uint16)
    up_page = np.ascontiguousarray(up_page, dtype=np.uint8)
    gate_page = np.ascontiguousarray(gate_page, dtype=np.uint8)
    out = np.empty(m, dtype=np.uint16)
    lib().v3o_partial_swiglu_int4(_p(x_f16), _p(up_page), _p(gate_page), _p(out), k, m)
    return out


def weighted_accumulate_f32(out: np.ndarray, expert_f16: np.ndarray, w: float) -> None:
    """kernels.rs:2000 weighted_accumulate_f32 CPU branch (in place)."""
    assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    e = np.ascontiguousarray(expert_f16, dtype=np.uint16)
    lib().v3o_weighted_accumulate_f32(_p(out), _p(e), float(w), out.size)


def weighted_accumulate_f16(out: np.ndarray, expert_f16: np.ndarray, w: float) -> None:
    """kernels.rs:1959 weighted_accumulate CPU branch: f16 accumulator bits, in place."""
    assert out.dtype == np.uint16 and out.flags["C_CONTIGUOUS"]
    e = np.ascontiguousarray(expert_f16, dtype=np.uint16)
    lib().v3o_weighted_accumulate_f16(_p(out), _p(e), float(w), out.size)


def router(x, w, w_dt, num_experts, hidden, top_k, mode, scaling=1.0, normalize=True,
           bias=None, nthreads=0):
    """kernels.rs:2307 run_router_with_scoring_and_bias CPU branch.

    Returns (ids uint16[k], weights f32[k], scores f32[E])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w)
    ids = np.empty(top_k, dtype=np.uint16)
    wts = np.empty(top_k, dtype=np.float32)
    scores = np.empty(num_experts, dtype=np.float32)
    b = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        b = _p(bias)
    rc = lib().v3o_router(_p(x), _p(w), w_dt, num_experts, hidden, top_k, mode, float(scaling),
                          int(bool(normalize)), b, _p(ids), _p(wts), _p(scores), nthreads)
    if rc != 0:
        raise ValueError("oracle router: bad arguments")
    return ids, wts, scores


def quantize_int4(w: np.ndarray, rows: int, cols: int, g: int = 32) -> np.ndarray:
    """kernels.rs:3778 quantize_weights_to_int4 (g generalised)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    pk, ng = (cols + 1) // 2, (cols + g - 1) // g
    out = np.zeros(rows * pk + rows * ng * 2, dtype=np.uint8)
    lib().v3o_quantize_int4(_p(w), rows, cols, g, _p(out))
    return out


def dequantize_int4(page, rows, cols, g, scale_dt) -> np.ndarray:
    """kernels.rs:3866 dequantize_int4_to_f32."""
    page = np.ascontiguousarray(page, dtype=np.uint8)
    out = np.empty(rows * cols, dtype=np.float32)
    lib().v3o_dequantize_int4(_p(page), rows, cols, g, scale_dt, _p(out))
    return out.reshape(rows, cols)


class _Matrix(C.Structure):
    _fields_ = [("pages", C.POINTER(C.c_void_p)), ("npages", C.c_size_t),
                ("rows_per_page", C.c_size_t)]


class _Expert(C.Structure):
    _fields_ = [("up", _Matrix), ("gate", _Matrix), ("down", _Matrix)]


def _expert_struct(pages_by_seg, rows_by_seg, keep):
    """pages_by_seg: 3 lists of uint8 page arrays (up, gate, down)."""
    ex = _Expert()
    for name, pages, rpp in zip(("up", "gate", "down"), pages_by_seg, rows_by_seg):
        arr = (C.c_void_p * len(pages))(*[p.ctypes.data for p in pages])
        keep.append(arr)
        keep.extend(pages)
        setattr(ex, name, _Matrix(C.cast(arr, C.POINTER(C.c_void_p)), len(pages), rpp))
    return ex


def moe_layer(x, hidden, inter, g, scale_dt, routed, ids, weights, shared, faithful=True,
              nthreads=0, shared_weights=None) -> np.ndarray:
    """engine.rs:5801 execute_expert x k + :6317 execute_shared_expert, summed in f32.

    routed: dict expert_id -> (pages_by_seg, rows_by_seg); only ids need to be present.
    shared: list of (pages_by_seg, rows_by_seg); shared_weights: their gates (None: 1.0)."""
    keep = []
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.uint16)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    n_routed = int(ids.max()) + 1 if ids.size else 0
    arr = (_Expert * max(n_routed, 1))()
    for e in set(int(i) for i in ids):
        pages, rows = routed[e]
        arr[e] = _expert_struct(pages, rows, keep)
    sh = (_Expert * max(len(shared), 1))()
    for s, (pages, rows) in enumerate(shared):
        sh[s] = _expert_struct(pages, rows, keep)
    out = np.empty(hidden, dtype=np.float32)
    sw = None if shared_weights is None else np.ascontiguousarray(shared_weights, np.float32)
    lib().v3o_moe_layer_w(_p(x), hidden, inter, g, scale_dt, C.cast(arr, C.c_void_p), _p(ids),
                          _p(weights), ids.size, C.cast(sh, C.c_void_p), len(shared),
                          None if sw is None else _p(sw), int(bool(faithful)), _p(out), nthreads)
    return out


# ---------------------------------------------------------------- either side of the MoE

def inv_rms(x, eps) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().v3o_inv_rms(_p(x), x.size, float(eps))


def rms_norm_f32(x, w_f16_bits, eps) -> np.ndarray:
    """vib3_rms_norm_f32 (kernels.cu:921): (x * inv_rms) * f32(w), x f32, w f16 bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w_f16_bits, dtype=np.uint16)
    out = np.empty_like(x)
    lib().v3o_rms_norm_f32(_p(x), x.size, _p(w), float(eps), _p(out))
    return out


def residual_add_f32(acc, lo) -> np.ndarray:
    out = np.array(acc, dtype=np.float32, copy=True)
    lo = np.ascontiguousarray(lo, dtype=np.float32)
    lib().v3o_residual_add_f32(_p(out), _p(lo), out.size)
    return out


def linear_row_f16(x, w_f16_bits) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w_f16_bits, dtype=np.uint16)
    return lib().v3o_linear_row_f16(_p(x), _p(w), x.size)


def sigmoid(g) -> float:
    return lib().v3o_sigmoid(float(g))


def e2m1(code: int) -> float:
    return lib().v3o_e2m1(code)


def e8m0(e: int) -> float:
    return lib().v3o_e8m0(e)


def matmul_mxfp4_acc(x, codes, scales, k, m, nthreads=0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    out = np.empty(m, dtype=np.float32)
    lib().v3o_matmul_mxfp4_acc(_p(x), _p(codes), _p(scales), k, m, _p(out), nthreads)
    return out


# ---------------------------------------------------------------- synthetic data

def synth_bytes(seed, stream, off, n) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    lib().v3o_synth_bytes(seed, stream, off, n, _p(out))
    return out


def synth_normal_array(seed, stream, off, n, sigma, dt) -> np.ndarray:
    out = np.empty(n, dtype=np.float32 if dt == F32 else np.uint16)
    lib().v3o_synth_normal_array(seed, stream, off, n, float(sigma), dt, _p(out))
    return out


def synth_int4_page(seed, stream, k, g, scale_dt, sigma, row_start, rows) -> np.ndarray:
    pk, ng = (k + 1) // 2, (k + g - 1) // g
    out = np.empty(rows * pk + rows * ng * 2, dtype=np.uint8)
    lib().v3o_synth_int4_page(seed, stream, k, g, scale_dt, float(sigma), row_start, rows, _p(out))
    return out


def synth_mxfp4_page(seed, stream, k, row_start, rows) -> np.ndarray:
    """MXFP4 page ([rows x k/2] codes, then [rows x k/32] E8M0 bytes) of logical matrix `stream`."""
    out = np.empty(rows * (k // 2) + rows * (k // 32), dtype=np.uint8)
    lib().v3o_synth_mxfp4_page(seed, stream, k, row_start, rows, _p(out))
    return out


def moe_mxfp4_batched(x, hidden, inter, pages, ids, weights, nthreads=0) -> np.ndarray:
    """Per-token restatement of the batched MXFP4 MoE (see cpu_ref.h); returns bf16 bits.

    x: [tokens, hidden] f32 (the bf16 activations, widened); pages: list over experts of
    (up, gate, down) uint8 pages; ids / weights: [tokens, top_k]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    tokens = x.shape[0]
    ids = np.ascontiguousarray(ids, dtype=np.uint16)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    top_k = ids.shape[1]
    keep = [np.ascontiguousarray(p, dtype=np.uint8) for trio in pages for p in trio]
    arr = (C.c_void_p * len(keep))(*[k.ctypes.data for k in keep])
    out = np.empty((tokens, hidden), dtype=np.uint16)
    lib().v3o_moe_mxfp4_batched(_p(x), tokens, hidden, inter, C.cast(arr, C.c_void_p),
                                len(pages), _p(ids), _p(weights), top_k, _p(out), nthreads)
    return out


# ---------------------------------------------------------------- NVFP4 fused MoE

def fp4_e8m0_of_amax(amax: float) -> int:
    return int(lib().v3o_fp4_e8m0_of_amax(float(amax)))


def e2m1_rne(v: float) -> int:
    return int(lib().v3o_e2m1_rne(float(v)))


def exp_cw(x: float) -> float:
    return float(lib().v3o_exp_cw(float(x)))


def fp4_quantize_act(x) -> tuple:
    """kernels.cu:3193 activation quantizer: (split-half codes, E8M0 scales)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = (x.size + 31) // 32
    codes = np.zeros(g * 16, dtype=np.uint8)
    sc = np.zeros(g, dtype=np.uint8)
    lib().v3o_fp4_quantize_act(_p(x), x.size, _p(codes), _p(sc))
    return codes, sc


def fp4_norm_inv(x, eps) -> float:
    """Inverse RMS in the order of kernels.cu:6610-6645 (correctly rounded 1/sqrt)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(np.float32(lib().v3o_fp4_norm_inv(_p(x), x.size, float(eps))))


def fused_rms_norm_quantize_fp4(x, w_f16_bits, eps, f16_out=False) -> tuple:
    """kernels.cu:6585 fused RMSNorm + FP4 quantize: (codes, scales[, f16 bits of the norm])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w_f16_bits, dtype=np.uint16)
    g = (x.size + 31) // 32
    codes = np.zeros(g * 16, dtype=np.uint8)
    sc = np.zeros(g, dtype=np.uint8)
    h = np.zeros(x.size, dtype=np.uint16) if f16_out else None
    lib().v3o_fused_rms_norm_quantize_fp4(_p(x), _p(w), x.size, float(eps), _p(codes), _p(sc),
                                          _p(h) if f16_out else None)
    return (codes, sc, h) if f16_out else (codes, sc)


def nvfp4_matvec(act_codes, act_scales, data, scales, m, k) -> np.ndarray:
    out = np.empty(m, dtype=np.float32)
    a = np.ascontiguousarray(act_codes, dtype=np.uint8)
    s = np.ascontiguousarray(act_scales, dtype=np.uint8)
    d = np.ascontiguousarray(data, dtype=np.uint8)
    w = np.ascontiguousarray(scales, dtype=np.uint16)
    lib().v3o_nvfp4_matvec(_p(a), _p(s), _p(d), _p(w), m, k, _p(out))
    return out


def moe_experts_fused(act_codes, act_scales, experts, weights, k_in, m_mid, m_out, out):
    """experts: per active expert ((up_data, up_scales), (gate_data, gate_scales),
    (down_data, down_scales)); out (f32 [m_out]) accumulated in place."""
    keep = []
    dp = (C.c_void_p * (3 * len(experts)))()
    sp = (C.c_void_p * (3 * len(experts)))()
    for e, mats in enumerate(experts):
        for s, (d, w) in enumerate(mats):
            d = np.ascontiguousarray(d, dtype=np.uint8)
            w = np.ascontiguousarray(w, dtype=np.uint16)
            keep += [d, w]
            dp[e * 3 + s] = d.ctypes.data
            sp[e * 3 + s] = w.ctypes.data
    wt = np.ascontiguousarray(weights, dtype=np.float32)
    a = np.ascontiguousarray(act_codes, dtype=np.uint8)
    sc = np.ascontiguousarray(act_scales, dtype=np.uint8)
    assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    lib().v3o_moe_experts_fused(_p(a), _p(sc), dp, sp, _p(wt), len(experts), k_in, m_mid, m_out,
                                _p(out))
    return out


def fp4_split_half(data) -> np.ndarray:
    d = np.array(data, dtype=np.uint8, copy=True)
    lib().v3o_fp4_split_half(_p(d), d.size)
    return d


def fp4_to_tiled(src, m, k) -> np.ndarray:
    s = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.zeros(m * k // 2, dtype=np.uint8)
    lib().v3o_fp4_to_tiled(_p(s), _p(dst), m, k)
    return dst


# ---------------------------------------------------------------- NVFP4 weight quantizers

def quantize_weights_to_nvfp4(w, rows, cols) -> np.ndarray:
    """kernels.rs:4085: row-major E2M1 codes (low nibble = even column), then f16 scales."""
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    assert w.size == rows * cols
    out = np.zeros(lib().v3o_nvfp4_page_bytes(rows, cols), dtype=np.uint8)
    lib().v3o_quantize_weights_to_nvfp4(_p(w), rows, cols, _p(out))
    return out


def quantize_half_to_nvfp4(bits, dt, rows, cols) -> np.ndarray:
    """kernels.rs:4172 (dt F16) / :4183 (dt BF16)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    out = np.zeros(lib().v3o_nvfp4_page_bytes(rows, cols), dtype=np.uint8)
    lib().v3o_quantize_half_to_nvfp4(_p(b), dt, rows, cols, _p(out))
    return out


def convert_int4_to_nvfp4(page, rows, cols, g) -> np.ndarray:
    """kernels.rs:3937: INT4 page (BF16 group scales) -> NVFP4 page (f16 block scales)."""
    p = np.ascontiguousarray(page, dtype=np.uint8).ravel()
    out = np.zeros(lib().v3o_nvfp4_page_bytes(rows, cols), dtype=np.uint8)
    lib().v3o_convert_int4_to_nvfp4(_p(p), p.size, rows, cols, g, _p(out))
    return out


def fp16_to_nvfp4_weight(w_f16_bits, m, k):
    """kernels.cu:6017: (row-major split-half codes [m*k/2], bf16 E8M0 scales [m*k/32])."""
    b = np.ascontiguousarray(w_f16_bits, dtype=np.uint16).ravel()
    data = np.zeros(m * k // 2, dtype=np.uint8)
    sc = np.zeros(m * (k // 32), dtype=np.uint16)
    lib().v3o_fp16_to_nvfp4_weight(_p(b), m, k, _p(data), _p(sc))
    return data, sc


def nvfp4_seq_matvec_f64(x, data, scales, m, k) -> np.ndarray:
    """f64 matvec of a row-major sequential NVFP4 matrix with full bf16 scales."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = np.ascontiguousarray(data, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    out = np.empty(m, dtype=np.float64)
    lib().v3o_nvfp4_seq_matvec_f64(_p(x), _p(d), _p(s), m, k, _p(out))
    return out


def nvfp4_page_matvec(act_codes, act_scales, data, scales, m, k, layout, full=False):
    """Block-scaled page GEMV; layout 0 row-major split-half, 1 tiled, 2 sequential."""
    a = np.ascontiguousarray(act_codes, dtype=np.uint8)
    s = np.ascontiguousarray(act_scales, dtype=np.uint8)
    d = np.ascontiguousarray(data, dtype=np.uint8)
    w = np.ascontiguousarray(scales, dtype=np.uint16)
    out = np.empty(m, dtype=np.float32)
    lib().v3o_nvfp4_page_matvec(_p(a), _p(s), _p(d), _p(w), m, k, layout, int(full), _p(out))
    return out


def nvfp4_page_swiglu(act_codes, act_scales, up, up_s, gate, gate_s, m, k, layout):
    a = np.ascontiguousarray(act_codes, dtype=np.uint8)
    s = np.ascontiguousarray(act_scales, dtype=np.uint8)
    arrs = [np.ascontiguousarray(v, dtype=t) for v, t in
            ((up, np.uint8), (up_s, np.uint16), (gate, np.uint8), (gate_s, np.uint16))]
    out = np.empty(m, dtype=np.float32)
    lib().v3o_nvfp4_page_swiglu(_p(a), _p(s), *[_p(v) for v in arrs], m, k, layout, _p(out))
    return out
