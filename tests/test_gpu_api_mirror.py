"""GPU parity of the Python mirror of the reference's Rust launcher API (vib3_amd/kernels.py,
kernels.rs names) against the CPU oracle, and BASELINE config c0 through it: one full-size
Mixtral expert (gate/up 14336 x 4096, down 4096 x 14336, INT4 g128, fp16 scales) as the
reference's public API runs it: partial_swiglu into an f16 h, then partial_matmul.

Bars as in test_gpu_kernels.py: f16 outputs within one f16 ulp of the oracle's rounded value
(plus 1e-5 of the largest |ref| for the fp32 summation order; 5e-5 for c0's down GEMV, whose
input is the heavy-tailed SwiGLU output); router ids bit-exact where the
k-th / (k+1)-th selection margin exceeds 1e-3, weights within 1e-5 relative."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 0x5EED0000


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def close16(got16, ref32, noise=1e-5):
    got = O.to_f32(got16.cpu().view(torch.int16).numpy().view(np.uint16), O.F16)
    ref16 = O.to_f32(O.f16_bits(ref32), O.F16)
    tol = np.abs(ref16) * 2.0 ** -10 + 2.0 ** -24 + noise * np.abs(ref32).max()
    bad = np.abs(got - ref16) > tol
    if bad.any():
        i = int(np.argmax(np.abs(got - ref16) / tol))
        _say(f"  {int(bad.sum())} outside the bar; worst at {i}: got {got[i]!r} ref {ref32[i]!r} "
             f"ref16 {ref16[i]!r} tol {tol[i]:.3e}; rel_l2 "
             f"{np.linalg.norm(got - ref32) / np.linalg.norm(ref32):.2e}")
    return bool(not bad.any()), got


def page(stream, k, m, g, sdt, sigma):
    host = O.synth_int4_page(SEED, stream, k, g, sdt, sigma, 0, m)
    return host, torch.from_numpy(host).cuda()


def x_f16(n, stream):
    bits = O.synth_normal_array(SEED, stream, 0, n, 1.0, O.F16)
    return O.to_f32(bits, O.F16), torch.from_numpy(bits.view(np.int16)).cuda().view(torch.float16)


def test_c0_mixtral_expert_through_public_api():
    """c0: x f16 [4096] ~N(0,1); gate/up [14336, 4096], down [4096, 14336], g128 fp16 scales
    ~|N(0, 0.02)|; out = down(silu(gate.x) * (up.x)) with the reference's f16 rounding of h
    and of the output (kernels.rs:3042, :2825)."""
    from vib3_amd import kernels as K
    from vib3_amd._lib import DT_F16
    _say("case: c0 full-size expert via partial_swiglu + partial_matmul")
    H, I, g = 4096, 14336, 128
    up_h, up = page(1, H, I, g, O.F16, 0.02)
    gate_h, gate = page(2, H, I, g, O.F16, 0.02)
    down_h, down = page(3, I, H, g, O.F16, 0.02)
    xh, x = x_f16(H, 4)
    h = torch.empty(I, dtype=torch.float16, device="cuda")
    K.partial_swiglu(x, up, gate, h, H, I, K.DType.INT4, group_size=g, scale_dtype=DT_F16)
    out = torch.empty(H, dtype=torch.float16, device="cuda")
    K.partial_matmul(h, down, out, I, H, K.DType.INT4, group_size=g, scale_dtype=DT_F16)
    torch.cuda.synchronize()
    ref_h = O.swiglu_int4_acc(xh, up_h, gate_h, H, I, g, O.F16)
    ok, got_h = close16(h, ref_h)
    assert ok
    # the down GEMV on the device's own h (an f16 vector both sides share), then end to end.
    # h is heavy-tailed (|h| up to ~300 beside values near 0), so the fp32 sums cancel more
    # than for N(0, 1) inputs: the summation-order allowance is the GEMV bar, 5e-5 of max|ref|
    ref_out = O.matmul_int4_acc(got_h, down_h, I, H, g, O.F16)
    ok, got = close16(out, ref_out, noise=5e-5)
    assert ok
    ref_full = O.matmul_int4_acc(O.to_f32(O.f16_bits(ref_h), O.F16), down_h, I, H, g, O.F16)
    rel = np.linalg.norm(got - ref_full) / np.linalg.norm(ref_full)
    _say(f"  c0 end-to-end rel_l2 {rel:.2e}")
    assert rel <= 1e-3


@pytest.mark.parametrize("k,m,sdt", [(7168, 256, O.BF16), (2048, 512, O.F16)])
def test_partial_matmul_and_f32_variants(k, m, sdt):
    """partial_matmul (f16 in) and partial_matmul_f32 / partial_swiglu_f32 (f32 in)."""
    from vib3_amd import kernels as K
    _say(f"case: mirror partial_matmul k={k} m={m}")
    g = 32
    w_h, w = page(10 + k, k, m, g, sdt, 0.02)
    xh, x = x_f16(k, 20 + k)
    out = torch.empty(m, dtype=torch.float16, device="cuda")
    K.partial_matmul(x, w, out, k, m, K.DType.INT4, group_size=g, scale_dtype=sdt)
    assert close16(out, O.matmul_int4_acc(xh, w_h, k, m, g, sdt))[0]
    x32 = torch.from_numpy(xh.astype(np.float32) * np.float32(0.37)).cuda()
    K.partial_matmul_f32(x32, w, out, k, m, K.DType.INT4, group_size=g, scale_dtype=sdt)
    assert close16(out, O.matmul_int4_acc(x32.cpu().numpy(), w_h, k, m, g, sdt))[0]
    u_h, u = page(30 + k, k, m, g, sdt, 0.02)
    K.partial_swiglu_f32(x32, u, w, out, k, m, K.DType.INT4, group_size=g, scale_dtype=sdt)
    assert close16(out, O.swiglu_int4_acc(x32.cpu().numpy(), u_h, w_h, k, m, g, sdt))[0]
    with pytest.raises(NotImplementedError):
        K.partial_matmul(x, w, out, k, m, K.DType.FP16)
    with pytest.raises(TypeError):
        K.partial_matmul_f32(x, w, out, k, m)  # f16 input to the f32 entry point


def test_reference_public_partial_matmul_defaults():
    """partial_matmul(..., DType::INT4) with the reference CPU path's defaults: g = 32 and BF16
    scales (kernels.rs:2733-2746, :2789), against v3o_partial_matmul_int4 (the oracle's public
    entry) bit for bit in f16 up to the one-ulp summation bar."""
    from vib3_amd import kernels as K
    _say("case: mirror partial_matmul defaults")
    k, m = 1024, 96
    w_h, w = page(50, k, m, 32, O.BF16, 0.03)
    xh, x = x_f16(k, 51)
    out = torch.empty(m, dtype=torch.float16, device="cuda")
    K.partial_matmul(x, w, out, k, m)
    ref = O.to_f32(O.partial_matmul_int4(O.f16_bits(xh), w_h, k, m), O.F16)
    got = O.to_f32(out.cpu().view(torch.int16).numpy().view(np.uint16), O.F16)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("E,k,scoring", [(384, 8, "sigmoid"), (8, 2, "softmax"), (300, 6, "softmax")])
def test_router_mirror(E, k, scoring):
    """run_router_with_scoring_and_bias, run_router_gpu_topk and run_router_gpu_topk_nosync
    (kernels.rs:2307, :1811, :1890) against the oracle's router."""
    from vib3_amd import kernels as K
    _say(f"case: mirror router E={E} k={k} {scoring}")
    D = 2048
    rng = np.random.default_rng(E)
    xh = O.to_f32(O.f16_bits(rng.normal(0, 1, D)), O.F16)
    w = rng.normal(0, 0.02, (E, D)).astype(np.float32)
    bias = rng.normal(0, 0.1, E).astype(np.float32) if scoring == "sigmoid" else None
    func = K.Sigmoid(2.827, True) if scoring == "sigmoid" else K.Softmax()
    mode, scale = (1, 2.827) if scoring == "sigmoid" else (0, 1.0)
    r_ids, r_wts, r_sc = O.router(xh, w, O.F32, E, D, k, mode, scale, True, bias)
    keys = r_sc.astype(np.float64)
    if mode == 1:
        keys = 1 / (1 + np.exp(-keys)) + bias
    s = np.sort(keys)[::-1]
    assert k == E or s[k - 1] - s[k] > 1e-3, "selection margin below 1e-3: choose another seed"
    x = torch.from_numpy(xh.astype(np.float32)).cuda()
    wt = torch.from_numpy(w).cuda()
    bt = torch.from_numpy(bias).cuda() if bias is not None else None
    pairs = K.run_router_with_scoring_and_bias(x, wt, E, D, k, func, correction_bias=bt)
    assert [p[0] for p in pairs] == r_ids.tolist()
    assert np.allclose([p[1] for p in pairs], r_wts, rtol=1e-5)
    ids = torch.empty(k, dtype=torch.int16, device="cuda")
    wts = torch.empty(k, dtype=torch.float32, device="cuda")
    sc = torch.empty(E, dtype=torch.float32, device="cuda")
    K.run_router_gpu_topk_nosync(x, wt, E, D, k, func, ids, wts, correction_bias=bt, scores_dev=sc)
    torch.cuda.synchronize()
    assert ids.cpu().numpy().view(np.uint16).tolist() == r_ids.tolist()
    # logits: fp32 dots of 2048 terms in another order (1e-5 of the largest logit)
    assert np.allclose(sc.cpu().numpy(), r_sc, rtol=0, atol=1e-5 * np.abs(r_sc).max())
    if bias is None:  # run_router_gpu_topk passes no bias (kernels.rs:1840)
        pairs = K.run_router_gpu_topk(x, wt, E, D, k, func)
        assert [p[0] for p in pairs] == r_ids.tolist()
