"""Host mirror of vib3's launcher API (src/compute/kernels.rs) over libvib3_hip.

Same function names, argument meaning and error behaviour as the reference launchers, with
torch tensors standing in for raw device pointers (``tensor.data_ptr()`` is what crosses the C
ABI). Every call runs the HIP kernels on the current torch stream of the tensor's device;
there is no CPU branch — a missing library or a CPU tensor raises.

Scale dtype: the reference CPU fallback decodes INT4 group scales as BF16
(kernels.rs:2789) while its GPU kernels decode FP16 (kernels.cu:45, :140). The functions here
take ``scale_dtype`` (default BF16, the CPU-fallback semantics the parity tests hold them to);
the reference GPU behaviour is ``scale_dtype=DT_F16``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import DT_BF16, DT_F16, DT_F32, ROUTER_SIGMOID, ROUTER_SOFTMAX

INT4_GROUP_SIZE = 32  # kernels.rs:3737


class DType:
    """Subset of core/types.rs:633 DType used by the expert path."""

    FP16 = 1
    BF16 = 2
    INT4 = 5
    NVFP4 = 7


@dataclass(frozen=True)
class Softmax:
    """kernels.rs:2226 RouterScoringFunc::Softmax."""


@dataclass(frozen=True)
class Sigmoid:
    """kernels.rs:2226 RouterScoringFunc::Sigmoid { scaling_factor, normalize }."""

    scaling_factor: float = 1.0
    normalize: bool = True


RouterScoringFunc = object  # Softmax() | Sigmoid(...)

_TORCH_DT = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}


def _dev(t: torch.Tensor, name: str) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor (no CPU fallback in vib3_amd)")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _act_dt(t: torch.Tensor, name: str) -> int:
    if t.dtype not in _TORCH_DT:
        raise TypeError(f"{name}: unsupported dtype {t.dtype}")
    return _TORCH_DT[t.dtype]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_int4(weight_dtype: int) -> None:
    if weight_dtype != DType.INT4:
        raise NotImplementedError("vib3_amd implements the INT4 expert path (DType.INT4)")


def partial_matmul(input: torch.Tensor, weight_page: torch.Tensor, output: torch.Tensor, k: int,
                   m_slice: int, weight_dtype: int = DType.INT4, group_size: int = INT4_GROUP_SIZE,
                   scale_dtype: int = DT_BF16) -> None:
    """kernels.rs:25 partial_matmul: output[m_slice] = weight_page[m_slice, k] . input[k].

    input f32/f16/bf16; output f16 or f32; weight_page = [m*ceil(k/2) nibbles][m*G*2 scales]."""
    _need_int4(weight_dtype)
    _lib.call("vib3_launch_partial_matmul_int4_ex", _dev(input, "input"), _act_dt(input, "input"),
              _dev(weight_page, "weight_page"), _dev(output, "output"),
              _act_dt(output, "output"), k, m_slice, group_size, scale_dtype, _stream(input))


def partial_matmul_f32(input, weight_page, output, k, m_slice, weight_dtype=DType.INT4,
                       group_size=INT4_GROUP_SIZE, scale_dtype=DT_BF16) -> None:
    """kernels.rs:375 partial_matmul_f32 (f32 input)."""
    if input.dtype != torch.float32:
        raise TypeError("partial_matmul_f32 takes an f32 input")
    partial_matmul(input, weight_page, output, k, m_slice, weight_dtype, group_size, scale_dtype)


def partial_swiglu(input: torch.Tensor, up_page: torch.Tensor, gate_page: torch.Tensor,
                   output: torch.Tensor, hidden_dim: int, m_slice: int,
                   weight_dtype: int = DType.INT4, swiglu_temps=None,
                   group_size: int = INT4_GROUP_SIZE, scale_dtype: int = DT_BF16) -> None:
    """kernels.rs:162 partial_swiglu: output = silu(gate . input) * (up . input), one launch.

    ``swiglu_temps`` is accepted for signature compatibility and unused: the fused kernel has no
    intermediates."""
    _need_int4(weight_dtype)
    _lib.call("vib3_launch_partial_swiglu_int4_ex", _dev(input, "input"), _act_dt(input, "input"),
              _dev(up_page, "up_page"), _dev(gate_page, "gate_page"), _dev(output, "output"),
              _act_dt(output, "output"), hidden_dim, m_slice, group_size, scale_dtype,
              _stream(input))


def partial_swiglu_f32(input, up_page, gate_page, output, hidden_dim, m_slice,
                       weight_dtype=DType.INT4, swiglu_temps=None, group_size=INT4_GROUP_SIZE,
                       scale_dtype=DT_BF16) -> None:
    """kernels.rs:459 partial_swiglu_f32 (f32 input)."""
    if input.dtype != torch.float32:
        raise TypeError("partial_swiglu_f32 takes an f32 input")
    partial_swiglu(input, up_page, gate_page, output, hidden_dim, m_slice, weight_dtype,
                   swiglu_temps, group_size, scale_dtype)


def weighted_accumulate_f32(output: torch.Tensor, expert_output: torch.Tensor, weight: float,
                            dim: int) -> None:
    """kernels.rs:2000 weighted_accumulate_f32: output_f32 += weight * expert_output (f16/f32)."""
    if output.dtype != torch.float32:
        raise TypeError("output must be f32")
    name = ("vib3_launch_weighted_accumulate_f32" if expert_output.dtype == torch.float16
            else "vib3_launch_weighted_accumulate_f32_f32")
    if expert_output.dtype not in (torch.float16, torch.float32):
        raise TypeError("expert_output must be f16 or f32")
    _lib.call(name, _dev(output, "output"), _dev(expert_output, "expert_output"), float(weight),
              dim, _stream(output))


def rms_norm_f32(input: torch.Tensor, output: torch.Tensor, weight: torch.Tensor, dim: int,
                 eps: float) -> None:
    """kernels.rs:1567 rms_norm_f32: output = input * inv_rms * weight (f32 in/out, f16 weight);
    output f16 gives kernels.rs:1604 rms_norm_f32_to_f16."""
    if input.dtype != torch.float32 or weight.dtype != torch.float16:
        raise TypeError("rms_norm_f32 takes an f32 input and f16 weights")
    if output.dtype == torch.float32:
        name = "vib3_launch_rms_norm_f32"
    elif output.dtype == torch.float16:
        name = "vib3_launch_rms_norm_f32_to_f16"
    else:
        raise TypeError("output must be f32 or f16")
    _lib.call(name, _dev(input, "input"), _dev(output, "output"), _dev(weight, "weight"), dim,
              float(eps), _stream(input))


def rms_norm_f32_to_f16(input, output, weight, dim, eps) -> None:
    """kernels.rs:1604."""
    if output.dtype != torch.float16:
        raise TypeError("output must be f16")
    rms_norm_f32(input, output, weight, dim, eps)


def residual_add_f32_f32(accumulator: torch.Tensor, layer_output: torch.Tensor, dim: int) -> None:
    """kernels.rs:2195: accumulator += layer_output (both f32)."""
    if accumulator.dtype != torch.float32 or layer_output.dtype != torch.float32:
        raise TypeError("residual_add_f32_f32 takes f32 tensors")
    _lib.call("vib3_launch_residual_add_f32_f32", _dev(accumulator, "accumulator"),
              _dev(layer_output, "layer_output"), dim, _stream(accumulator))


def sigmoid_gated_accumulate_f32(output: torch.Tensor, expert_output: torch.Tensor,
                                 gate_dev: torch.Tensor, dim: int) -> None:
    """kernels.rs:2080: output += sigmoid(gate_dev[0]) * expert_output (f16)."""
    if output.dtype != torch.float32 or expert_output.dtype != torch.float16 or \
            gate_dev.dtype != torch.float32:
        raise TypeError("sigmoid_gated_accumulate_f32 takes f32 output/gate and f16 expert output")
    _lib.call("vib3_launch_sigmoid_gated_accumulate_f32", _dev(output, "output"),
              _dev(expert_output, "expert_output"), _dev(gate_dev, "gate_dev"), dim,
              _stream(output))


def _scoring(scoring_func) -> Tuple[int, float, int]:
    if isinstance(scoring_func, Sigmoid):
        return ROUTER_SIGMOID, float(scoring_func.scaling_factor), int(scoring_func.normalize)
    if isinstance(scoring_func, Softmax) or scoring_func is None:
        return ROUTER_SOFTMAX, 1.0, 1
    raise TypeError(f"unknown scoring function {scoring_func!r}")


class RouterWorkspace:
    """Device workspace of the one-launch router (completion counter + scratch), zeroed once."""

    def __init__(self, num_experts: int, device) -> None:
        n = _lib.load().vib3_router_workspace_bytes(num_experts)
        self.buf = torch.zeros(n, dtype=torch.uint8, device=device)
        self.num_experts = num_experts


def run_router_gpu_topk_nosync(hidden_state: torch.Tensor, router_weights: torch.Tensor,
                               num_experts: int, hidden_dim: int, top_k: int, scoring_func,
                               topk_ids_dev: torch.Tensor, topk_weights_dev: torch.Tensor,
                               correction_bias: Optional[torch.Tensor] = None,
                               scores_dev: Optional[torch.Tensor] = None,
                               workspace: Optional[RouterWorkspace] = None) -> None:
    """kernels.rs:1890 run_router_gpu_topk_nosync: ids/weights stay on the device."""
    mode, scale, norm = _scoring(scoring_func)
    if workspace is None or workspace.num_experts < num_experts:
        workspace = RouterWorkspace(num_experts, hidden_state.device)
    if topk_ids_dev.dtype not in (torch.int16, torch.uint16):
        raise TypeError("topk_ids_dev must be a 16-bit tensor")
    bias_p = _dev(correction_bias, "correction_bias") if correction_bias is not None else None
    scores_p = _dev(scores_dev, "scores_dev") if scores_dev is not None else None
    _lib.call("vib3_launch_router_topk_ex", _dev(hidden_state, "hidden_state"),
              _act_dt(hidden_state, "hidden_state"), _dev(router_weights, "router_weights"),
              _act_dt(router_weights, "router_weights"), bias_p, hidden_dim, num_experts, top_k,
              mode, scale, norm, scores_p, _dev(topk_ids_dev, "topk_ids_dev"),
              _dev(topk_weights_dev, "topk_weights_dev"), workspace.buf.data_ptr(),
              _stream(hidden_state))


def run_router_with_scoring_and_bias(hidden_state: torch.Tensor, router_weights: torch.Tensor,
                                     num_experts: int, hidden_dim: int, top_k: int,
                                     scoring_func=Softmax(), scores_dev=None,
                                     correction_bias: Optional[torch.Tensor] = None,
                                     workspace: Optional[RouterWorkspace] = None
                                     ) -> List[Tuple[int, float]]:
    """kernels.rs:2307: route on the device, then copy the k (id, weight) pairs to the host
    (one small D2H, as run_router_gpu_topk does at kernels.rs:1859-1873)."""
    dev = hidden_state.device
    ids = torch.empty(top_k, dtype=torch.int16, device=dev)
    wts = torch.empty(top_k, dtype=torch.float32, device=dev)
    run_router_gpu_topk_nosync(hidden_state, router_weights, num_experts, hidden_dim, top_k,
                               scoring_func, ids, wts, correction_bias, scores_dev, workspace)
    ids_h = ids.cpu().numpy().view("uint16").tolist()
    return list(zip(ids_h, wts.cpu().tolist()))


def router_gemv(hidden_state: torch.Tensor, router_weights: torch.Tensor, scores: torch.Tensor,
                hidden_dim: int, num_experts: int) -> None:
    """cuda_ffi.rs:267 vib3_launch_router_gemv: f16 h x f16 W -> f32 scores on the device, the
    GEMV step of gpu_run_router (kernels.rs:2445-2465)."""
    if hidden_state.dtype != torch.float16 or router_weights.dtype != torch.float16:
        raise TypeError("router_gemv takes f16 hidden_state and f16 router_weights")
    if scores.dtype != torch.float32 or scores.numel() < num_experts:
        raise ValueError("scores must be f32 with at least num_experts elements")
    _lib.call("vib3_launch_router_gemv", _dev(hidden_state, "hidden_state"),
              _dev(router_weights, "router_weights"), _dev(scores, "scores"), hidden_dim,
              num_experts, _stream(hidden_state))


def run_router_gpu_topk(hidden_state, router_weights, num_experts, hidden_dim, top_k,
                        scoring_func, scores_dev=None, topk_ids_dev=None, topk_weights_dev=None):
    """kernels.rs:1811 run_router_gpu_topk (bias always NULL there)."""
    return run_router_with_scoring_and_bias(hidden_state, router_weights, num_experts, hidden_dim,
                                            top_k, scoring_func, scores_dev)


# ---------------------------------------------------------------- NVFP4 fused MoE

def quantize_activation_fp4(input: torch.Tensor, act_fp4: torch.Tensor, act_scales: torch.Tensor,
                            k: int) -> None:
    """kernels.rs:785 quantize_activation_fp4 (and :1486 _fast): f32 [k] -> split-half E2M1
    codes [k/2] (16-byte aligned) + E8M0 scales [k/32]."""
    if input.dtype != torch.float32:
        raise TypeError("quantize_activation_fp4 takes an f32 input")
    _lib.call("vib3_launch_quantize_activation_fp4", _dev(input, "input"),
              _dev(act_fp4, "act_fp4"), _dev(act_scales, "act_scales"), k, _stream(input))


quantize_activation_fp4_fast = quantize_activation_fp4


def fused_rms_norm_quantize_fp4(input: torch.Tensor, norm_weight: torch.Tensor,
                                act_fp4: torch.Tensor, act_scales: torch.Tensor,
                                opt_f16_out, k: int, eps: float) -> None:
    """kernels.rs:1641 fused_rms_norm_quantize_fp4: RMSNorm of the f32 hidden state [k] with
    f16 weights, then split-half E2M1 codes [k/2] + E8M0 scales [k/32]; opt_f16_out (an f16
    tensor [k], or None) receives the normalised values."""
    if input.dtype != torch.float32 or norm_weight.dtype != torch.float16:
        raise TypeError("fused_rms_norm_quantize_fp4 takes an f32 input and f16 weights")
    _lib.call("vib3_launch_fused_rms_norm_quantize_fp4", _dev(input, "input"),
              _dev(norm_weight, "norm_weight"), _dev(act_fp4, "act_fp4"),
              _dev(act_scales, "act_scales"),
              None if opt_f16_out is None else _dev(opt_f16_out, "opt_f16_out"), k, eps,
              _stream(input))


def moe_prewarm_gpu_bufs(m_mid: int, k_mid: int) -> None:
    """cuda_ffi.rs:1026 vib3_moe_prewarm_gpu_bufs: the fused MoE's intermediate buffer on the
    current device (the one allocation of this path; call before graph capture)."""
    _lib.call("vib3_moe_prewarm_gpu_bufs", m_mid, k_mid)


def _nvfp4_data_bytes(k: int, m: int) -> int:
    return ((k + 1) // 2) * m


def moe_experts_fused(act_fp4: torch.Tensor, act_scales: torch.Tensor,
                      expert_pages: Sequence[Tuple[int, int, int, float]], k_in: int, m_mid: int,
                      m_out: int, layer_output: torch.Tensor) -> None:
    """kernels.rs:1010 moe_experts_fused: expert_pages = (up_page, gate_page, down_page, weight)
    with device addresses of tiled split-half NVFP4 pages (scales after the data); at most 8
    are used; layer_output (f32 [m_out]) is accumulated."""
    n = min(len(expert_pages), 8)
    if n == 0:
        raise ValueError("moe_experts_fused needs at least one expert")
    arr = lambda: (C.c_void_p * 8)()
    uw, us, gw, gs, dw, ds = arr(), arr(), arr(), arr(), arr(), arr()
    w = (C.c_float * 8)()
    up_sz, down_sz = _nvfp4_data_bytes(k_in, m_mid), _nvfp4_data_bytes(m_mid, m_out)
    for i, (up, gate, down, wt) in enumerate(expert_pages[:n]):
        uw[i], us[i] = up, up + up_sz
        gw[i], gs[i] = gate, gate + up_sz
        dw[i], ds[i] = down, down + down_sz
        w[i] = wt
    _lib.call("vib3_launch_moe_experts_fused", _dev(act_fp4, "act_fp4"),
              _dev(act_scales, "act_scales"), uw, us, gw, gs, dw, ds, w, n, k_in, m_mid, m_mid,
              m_out, _dev(layer_output, "layer_output"), _stream(layer_output))


def moe_experts_fused_gpu(act_fp4: torch.Tensor, act_scales: torch.Tensor,
                          page_table: torch.Tensor, expert_ids: torch.Tensor,
                          expert_weights: torch.Tensor, moe_layer: int, num_experts_total: int,
                          num_active: int, k_in: int, m_mid: int, m_out: int,
                          layer_output: torch.Tensor) -> None:
    """kernels.rs:1091 moe_experts_fused_gpu: ids / weights and the page table
    u64[layers][experts][3] stay on the device (no host sync)."""
    _lib.call("vib3_launch_moe_experts_fused_gpu", _dev(act_fp4, "act_fp4"),
              _dev(act_scales, "act_scales"), _dev(page_table, "page_table"),
              _dev(expert_ids, "expert_ids"), _dev(expert_weights, "expert_weights"), moe_layer,
              num_experts_total, num_active, k_in, m_mid, m_mid, m_out,
              _dev(layer_output, "layer_output"), _stream(layer_output))


def _page_scales(page: torch.Tensor, k: int, m_slice: int) -> int:
    """Device address of a page's scales: after its packed codes (kernels.rs:821-860)."""
    return _dev(page, "page") + _nvfp4_data_bytes(k, m_slice)


def _need_f32(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be an f32 tensor")


def gemv_mma_nvfp4_preq(act_fp4: torch.Tensor, act_scales: torch.Tensor,
                        weight_page: torch.Tensor, output: torch.Tensor, k: int,
                        m_slice: int) -> None:
    """kernels.rs:821 gemv_mma_nvfp4_preq: pre-quantized activation times a row-major
    split-half NVFP4 page -> f32 [m_slice] (also :1200 gemv_mma_nvfp4_preq_fast)."""
    _need_f32(output, "output")
    _lib.call("vib3_launch_gemv_mma_nvfp4_preq", _dev(act_fp4, "act_fp4"),
              _dev(act_scales, "act_scales"), _dev(weight_page, "weight_page"),
              _page_scales(weight_page, k, m_slice), _dev(output, "output"), k, m_slice,
              _stream(output))


gemv_mma_nvfp4_preq_fast = gemv_mma_nvfp4_preq


def fused_swiglu_mma_nvfp4_preq(act_fp4: torch.Tensor, act_scales: torch.Tensor,
                                up_page: torch.Tensor, gate_page: torch.Tensor,
                                output: torch.Tensor, k: int, m_slice: int) -> None:
    """kernels.rs:862 fused_swiglu_mma_nvfp4_preq: (g * sigmoid(g)) * u of two page GEMVs,
    f32 [m_slice] (also :1520 fused_swiglu_mma_nvfp4_preq_fast)."""
    _need_f32(output, "output")
    _lib.call("vib3_launch_fused_swiglu_mma_nvfp4_preq", _dev(act_fp4, "act_fp4"),
              _dev(act_scales, "act_scales"), _dev(up_page, "up_page"),
              _page_scales(up_page, k, m_slice), _dev(gate_page, "gate_page"),
              _page_scales(gate_page, k, m_slice), _dev(output, "output"), k, m_slice,
              _stream(output))


fused_swiglu_mma_nvfp4_preq_fast = fused_swiglu_mma_nvfp4_preq


def gemv_mma_nvfp4(input: torch.Tensor, weight_page: torch.Tensor, output: torch.Tensor,
                   k: int, m_slice: int) -> None:
    """kernels.rs:696 gemv_mma_nvfp4: f32 input (quantized to FP4 in the kernel) times a
    sequential-nibble NVFP4 page -> f32."""
    _need_f32(input, "input")
    _need_f32(output, "output")
    _lib.call("vib3_launch_gemv_mma_nvfp4", _dev(input, "input"), _dev(weight_page, "weight_page"),
              _page_scales(weight_page, k, m_slice), _dev(output, "output"), k, m_slice,
              _stream(output))


def fused_swiglu_mma_nvfp4(input: torch.Tensor, up_page: torch.Tensor, gate_page: torch.Tensor,
                           output: torch.Tensor, k: int, m_slice: int) -> None:
    """kernels.rs:742 fused_swiglu_mma_nvfp4."""
    _need_f32(input, "input")
    _need_f32(output, "output")
    _lib.call("vib3_launch_fused_swiglu_mma_nvfp4", _dev(input, "input"), _dev(up_page, "up_page"),
              _page_scales(up_page, k, m_slice), _dev(gate_page, "gate_page"),
              _page_scales(gate_page, k, m_slice), _dev(output, "output"), k, m_slice,
              _stream(output))


def partial_matmul_nvfp4_f32(input: torch.Tensor, weight_page: torch.Tensor,
                             output: torch.Tensor, k: int, m_slice: int) -> None:
    """kernels.rs:652 partial_matmul_nvfp4_f32: f32 input times a sequential NVFP4 page with
    bf16 block scales, f32 output (vib3_launch_partial_matmul_nvfp4_f32out, block 32)."""
    _need_f32(input, "input")
    _need_f32(output, "output")
    _lib.call("vib3_launch_partial_matmul_nvfp4_f32out", _dev(input, "input"),
              _dev(weight_page, "weight_page"), _page_scales(weight_page, k, m_slice),
              _dev(output, "output"), k, m_slice, 32, _stream(output))


def partial_swiglu_f32_f32out(input: torch.Tensor, up_page: torch.Tensor,
                              gate_page: torch.Tensor, output: torch.Tensor, hidden_dim: int,
                              m_slice: int) -> None:
    """kernels.rs:604 partial_swiglu_f32_f32out (NVFP4 pages): silu(g) * u in f32."""
    _need_f32(input, "input")
    _need_f32(output, "output")
    _lib.call("vib3_launch_fused_swiglu_nvfp4_f32out", _dev(input, "input"),
              _dev(up_page, "up_page"), _page_scales(up_page, hidden_dim, m_slice),
              _dev(gate_page, "gate_page"), _page_scales(gate_page, hidden_dim, m_slice),
              _dev(output, "output"), hidden_dim, m_slice, 32, _stream(output))


def expert_batched(act_fp4: torch.Tensor, act_scales: torch.Tensor, up_page: torch.Tensor,
                   gate_page: torch.Tensor, down_page: torch.Tensor, layer_output: torch.Tensor,
                   expert_weight: float, k_in: int, m_mid: int, m_out: int) -> None:
    """kernels.rs:947 expert_batched: one expert over tiled split-half pages, layer_output
    (f32 [m_out]) += expert_weight * down(quantized SwiGLU(up, gate))."""
    _need_f32(layer_output, "layer_output")
    _lib.call("vib3_launch_expert_batched", _dev(act_fp4, "act_fp4"),
              _dev(act_scales, "act_scales"), _dev(up_page, "up_page"),
              _page_scales(up_page, k_in, m_mid), _dev(gate_page, "gate_page"),
              _page_scales(gate_page, k_in, m_mid), _dev(down_page, "down_page"),
              _page_scales(down_page, m_mid, m_out), _dev(layer_output, "layer_output"),
              float(expert_weight), k_in, m_mid, m_mid, m_out, _stream(layer_output))


def fp16_to_nvfp4_weight(input: torch.Tensor, m: int, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """kernels.rs:1161 fp16_to_nvfp4_weight: f16 [m, k] -> (row-major split-half codes
    [m * k / 2], bf16 E8M0 scales [m * k / 32])."""
    if input.dtype != torch.float16:
        raise TypeError("fp16_to_nvfp4_weight takes an f16 tensor")
    data = torch.empty(m * k // 2, dtype=torch.uint8, device=input.device)
    scales = torch.empty(m * k // 32, dtype=torch.int16, device=input.device)
    _lib.call("vib3_launch_fp16_to_nvfp4_weight", _dev(input, "input"), _dev(data, "data"),
              _dev(scales, "scales"), m, k, _stream(input))
    return data, scales


def repack_weights_inplace(weight_data: torch.Tensor, weight_data_bytes: int) -> None:
    """kernels.rs:915: sequential -> split-half nibble order, in place."""
    _lib.call("vib3_launch_repack_weights_inplace", _dev(weight_data, "weight_data"),
              weight_data_bytes, _stream(weight_data))


def repack_row_to_tiled(weight_data: torch.Tensor, temp_buf: torch.Tensor, m_slice: int,
                        k: int) -> None:
    """kernels.rs:1289: row-major split-half [m][k/2] -> 16x64 tiles, through temp_buf."""
    _lib.call("vib3_launch_repack_row_to_tiled", _dev(weight_data, "weight_data"),
              _dev(temp_buf, "temp_buf"), m_slice, k, _stream(weight_data))
