"""GPU parity of the single-page launchers against the CPU oracle (through the C ABI).

Bar: integer/byte outputs bit-exact; f32 GEMV outputs rel-L2 <= 5e-5 against the oracle's fp32
accumulators (only the summation order differs: the oracle's sequential fp32 sum over k <= 16384
terms carries ~1e-5 relative error of its own); f16 outputs within 1 f16 ulp of the oracle's
rounded value; router ids bit-exact where the k-th/(k+1)-th selection margin exceeds 1e-3.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _lib():
    from vib3_amd import _lib
    return _lib


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def close16(out16, ref):
    """f16 device output vs the oracle's f32 accumulators: within one f16 ulp of the rounded
    reference plus the fp32 summation-order noise (1e-5 of the largest |ref|)."""
    got = O.to_f32(out16.cpu().numpy().view(np.uint16), O.F16)
    ref16 = O.to_f32(O.f16_bits(ref), O.F16)
    tol = np.abs(ref16) * 2.0 ** -10 + 2.0 ** -24 + 1e-5 * np.abs(ref).max()
    return bool(np.all(np.abs(got - ref16) <= tol))


def synth_page(seed, stream, k, m, g, sdt, sigma=0.02):
    return O.synth_int4_page(seed, stream, k, g, sdt, sigma, 0, m)


def act(n, dt, seed=7, stream=11):
    """Activation as (device tensor, host f32 copy)."""
    bits = O.synth_normal_array(seed, stream, 0, n, 1.0, dt)
    host = O.to_f32(bits, dt) if dt != O.F32 else bits
    t = _dev(bits)
    if dt == O.F16:
        t = t.view(torch.float16)
    elif dt == O.BF16:
        t = t.view(torch.bfloat16)
    return t, host


# ---------------------------------------------------------------- generator

def test_synth_device_matches_oracle():
    L = _lib()
    _say("case: synth bytes/normal/int4 page")
    n = 100003
    buf = torch.empty(n, dtype=torch.uint8, device="cuda")
    L.call("vib3_synth_bytes", buf.data_ptr(), n, 5, 77, 3, _stream())
    assert np.array_equal(buf.cpu().numpy(), O.synth_bytes(5, 77, 3, n))
    for dt in (O.F32, O.F16, O.BF16):
        t = torch.empty(n * (4 if dt == O.F32 else 2), dtype=torch.uint8, device="cuda")
        L.call("vib3_synth_normal", t.data_ptr(), dt, n, 5, 78, 10, 0.37, _stream())
        ref = O.synth_normal_array(5, 78, 10, n, 0.37, dt)
        assert np.array_equal(t.cpu().numpy().view(ref.dtype), ref)
    for sdt in (O.F16, O.BF16):
        k, m, g = 512, 24, 32
        ref = O.synth_int4_page(9, 4, k, g, sdt, 0.01, 16, m)
        t = torch.empty(ref.size, dtype=torch.uint8, device="cuda")
        L.call("vib3_synth_int4_page", t.data_ptr(), 9, 4, k, g, sdt, 0.01, 16, m, _stream())
        assert np.array_equal(t.cpu().numpy(), ref)


# ---------------------------------------------------------------- reference KATs on the GPU

def test_kat_int4_matmul_on_gpu():
    """integration_test.rs:1709 and :1788 through vib3_launch_partial_matmul_int4_ex."""
    L = _lib()
    _say("case: KAT int4 (k=4, k=2, generic kernel)")
    page = _dev(np.array([0x89, 0x88, 0x98, 0x88, 0x80, 0x3F, 0x80, 0x3F], dtype=np.uint8))
    x = _dev(O.f16_bits([1.0, 2.0, 3.0, 4.0]))
    out = torch.zeros(2, dtype=torch.int16, device="cuda")
    L.call("vib3_launch_partial_matmul_int4_ex", x.data_ptr(), L.DT_F16, page.data_ptr(),
           out.data_ptr(), L.DT_F16, 4, 2, 32, L.DT_BF16, _stream())
    assert O.to_f32(out.cpu().numpy().view(np.uint16), O.F16).tolist() == [1.0, 2.0]
    page = _dev(np.array([0xAA, 0x00, 0x3F], dtype=np.uint8))
    x = _dev(O.f16_bits([3.0, 7.0]))
    out = torch.zeros(1, dtype=torch.int16, device="cuda")
    L.call("vib3_launch_partial_matmul_int4_ex", x.data_ptr(), L.DT_F16, page.data_ptr(),
           out.data_ptr(), L.DT_F16, 2, 1, 32, L.DT_BF16, _stream())
    assert O.to_f32(out.cpu().numpy().view(np.uint16), O.F16).tolist() == [10.0]


# ---------------------------------------------------------------- GEMV / SwiGLU parity

GEMV_TOL = 5e-5  # rel-L2, fp32 summation-order noise

GEMV_CASES = [
    # k, m, g, scale dtype, activation dtype
    (7168, 96, 32, O.BF16, O.BF16),     # Kimi gate/up rows (NCH=4, 224 chunks)
    (2048, 130, 32, O.BF16, O.F16),     # Kimi down rows (NCH=1), ragged m
    (4096, 64, 128, O.F16, O.F16),      # Mixtral gate/up, g=128 fp16 scales
    (14336, 40, 128, O.F16, O.F16),     # Mixtral down: k split over 2 waves
    (7168, 33, 32, O.BF16, O.F32),      # f32 activations (hi/lo split path)
    (1024, 7, 64, O.BF16, O.BF16),
    (96, 5, 32, O.BF16, O.F32),         # k % 64 != 0 (partial chunk slot)
    (100, 3, 32, O.BF16, O.F16),        # k % 32 != 0 -> generic kernel
    (31, 4, 32, O.F16, O.F32),          # odd k -> generic kernel
]


@pytest.mark.parametrize("k,m,g,sdt,adt", GEMV_CASES)
def test_partial_matmul_parity(k, m, g, sdt, adt):
    L = _lib()
    _say(f"case: partial_matmul k={k} m={m} g={g} sdt={sdt} adt={adt}")
    page = synth_page(0x5EED0000, 1000 + k, k, m, g, sdt)
    xt, xh = act(k, adt)
    dpage = _dev(page)
    out32 = torch.empty(m, dtype=torch.float32, device="cuda")
    out16 = torch.empty(m, dtype=torch.int16, device="cuda")
    for out, odt in ((out32, L.DT_F32), (out16, L.DT_F16)):
        L.call("vib3_launch_partial_matmul_int4_ex", xt.data_ptr(), adt, dpage.data_ptr(),
               out.data_ptr(), odt, k, m, g, sdt, _stream())
    ref = O.matmul_int4_acc(xh, page, k, m, g, sdt)
    got32 = out32.cpu().numpy()
    assert rel_l2(got32, ref) <= GEMV_TOL
    # the f16 output is the kernel's own f32 result rounded to nearest even
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), O.f16_bits(got32))
    assert close16(out16, ref)


@pytest.mark.parametrize("k,m,g,sdt,adt", GEMV_CASES)
def test_partial_swiglu_parity(k, m, g, sdt, adt):
    L = _lib()
    _say(f"case: partial_swiglu k={k} m={m} g={g} sdt={sdt} adt={adt}")
    up = synth_page(0x5EED0000, 2000 + k, k, m, g, sdt)
    gate = synth_page(0x5EED0000, 3000 + k, k, m, g, sdt)
    xt, xh = act(k, adt)
    dup, dgate = _dev(up), _dev(gate)
    out = torch.empty(m, dtype=torch.float32, device="cuda")
    L.call("vib3_launch_partial_swiglu_int4_ex", xt.data_ptr(), adt, dup.data_ptr(),
           dgate.data_ptr(), out.data_ptr(), L.DT_F32, k, m, g, sdt, _stream())
    ref = O.swiglu_int4_acc(xh, up, gate, k, m, g, sdt)
    assert rel_l2(out.cpu().numpy(), ref) <= GEMV_TOL


def test_invalid_scales_decode_as_one_eighth():
    L = _lib()
    _say("case: invalid scales")
    k, m = 64, 4
    data = np.full(m * 32, 0x99, dtype=np.uint8)
    sc = np.array([0x0000, 0xBF80, 0x7FC0, 0x7F80] * 2, dtype=np.uint16).reshape(2, m).T.copy()
    page = np.concatenate([data, sc.ravel().view(np.uint8)])
    xt, xh = act(k, O.F32)
    x1 = torch.ones(k, dtype=torch.float32, device="cuda")
    out = torch.empty(m, dtype=torch.float32, device="cuda")
    dpage = _dev(page)
    L.call("vib3_launch_partial_matmul_int4_ex", x1.data_ptr(), L.DT_F32, dpage.data_ptr(),
           out.data_ptr(), L.DT_F32, k, m, 32, L.DT_BF16, _stream())
    assert out.cpu().numpy().tolist() == [8.0] * 4


def test_empty_and_bad_arguments():
    L = _lib()
    _say("case: empty/bad args")
    lib = L.load()
    x = torch.zeros(64, dtype=torch.float32, device="cuda")
    page = torch.zeros(64, dtype=torch.uint8, device="cuda")
    out = torch.zeros(1, dtype=torch.float32, device="cuda")
    assert lib.vib3_launch_partial_matmul_int4_ex(x.data_ptr(), L.DT_F32, page.data_ptr(),
                                                  out.data_ptr(), L.DT_F32, 64, 0, 32,
                                                  L.DT_BF16, _stream()) == 0
    assert lib.vib3_launch_partial_matmul_int4_ex(x.data_ptr(), 9, page.data_ptr(),
                                                  out.data_ptr(), L.DT_F32, 64, 1, 32,
                                                  L.DT_BF16, _stream()) == -1
    assert lib.vib3_launch_partial_matmul_int4_ex(None, L.DT_F32, page.data_ptr(),
                                                  out.data_ptr(), L.DT_F32, 64, 1, 32,
                                                  L.DT_BF16, _stream()) == -3
    assert lib.vib3_launch_partial_matmul_int4_ex(x.data_ptr(), L.DT_F32, page.data_ptr(),
                                                  out.data_ptr(), L.DT_F32, 0, 1, 32,
                                                  L.DT_BF16, _stream()) == -2


# ---------------------------------------------------------------- reference-compatible launchers

def test_legacy_int4_launchers_fp16_scales():
    """vib3_launch_partial_matmul_int4(_f32) and fused_swiglu_int4_f32 decode FP16 scales like
    the reference GPU kernels (kernels.cu:45, :140); outputs are f16."""
    L = _lib()
    _say("case: legacy int4 launchers")
    k, m, g = 4096, 200, 32
    up = synth_page(1, 11, k, m, g, O.F16)
    gate = synth_page(1, 12, k, m, g, O.F16)
    pk = k // 2
    dup, dgate = _dev(up), _dev(gate)
    x16, x16h = act(k, O.F16)
    x32, x32h = act(k, O.F32)
    out = torch.empty(m, dtype=torch.int16, device="cuda")
    L.call("vib3_launch_partial_matmul_int4", x16.data_ptr(), dup.data_ptr(),
           dup.data_ptr() + pk * m, out.data_ptr(), k, m, g, _stream())
    assert close16(out, O.matmul_int4_acc(x16h, up, k, m, g, O.F16))
    L.call("vib3_launch_partial_matmul_int4_f32", x32.data_ptr(), dup.data_ptr(),
           dup.data_ptr() + pk * m, out.data_ptr(), k, m, g, _stream())
    assert close16(out, O.matmul_int4_acc(x32h, up, k, m, g, O.F16))
    L.call("vib3_launch_fused_swiglu_int4_f32", x32.data_ptr(), dup.data_ptr(),
           dup.data_ptr() + pk * m, dgate.data_ptr(), dgate.data_ptr() + pk * m, out.data_ptr(),
           k, m, g, _stream())
    assert close16(out, O.swiglu_int4_acc(x32h, up, gate, k, m, g, O.F16))


def test_silu_mul_and_weighted_accumulate():
    L = _lib()
    _say("case: silu_mul / weighted_accumulate")
    n = 5000
    a = O.f16_bits(np.random.default_rng(1).normal(0, 3, n))
    b = O.f16_bits(np.random.default_rng(2).normal(0, 3, n))
    da, db = _dev(a), _dev(b)
    out = torch.empty(n, dtype=torch.int16, device="cuda")
    L.call("vib3_launch_silu_mul", da.data_ptr(), db.data_ptr(), out.data_ptr(), n, _stream())
    af, bf = O.to_f32(a, O.F16), O.to_f32(b, O.F16)
    ref = O.to_f32(O.f16_bits((af / (1 + np.exp(-af.astype(np.float64)))) * bf), O.F16)
    got = O.to_f32(out.cpu().numpy().view(np.uint16), O.F16)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2 ** -10 + 2 ** -24)
    acc = np.random.default_rng(3).normal(0, 1, n).astype(np.float32)
    dacc = _dev(acc)
    L.call("vib3_launch_weighted_accumulate_f32", dacc.data_ptr(), da.data_ptr(), 0.37, n,
           _stream())
    ref = acc.copy()
    O.weighted_accumulate_f32(ref, a, 0.37)
    assert np.array_equal(dacc.cpu().numpy(), ref)  # same rounded mul then add
    e32 = np.random.default_rng(4).normal(0, 1, n).astype(np.float32)
    de = _dev(e32)
    L.call("vib3_launch_weighted_accumulate_f32_f32", dacc.data_ptr(), de.data_ptr(), -1.5, n,
           _stream())
    ref = ref + np.float32(-1.5) * e32
    assert np.array_equal(dacc.cpu().numpy(), ref.astype(np.float32))
    # f16 accumulator (kernels.rs:1959) and the device-scalar weight (cuda_ffi.rs:222)
    o16 = O.f16_bits(np.random.default_rng(5).normal(0, 2, n))
    do16 = _dev(o16)
    L.call("vib3_launch_weighted_accumulate", do16.data_ptr(), da.data_ptr(), 0.37, n, _stream())
    ref16 = o16.copy()
    O.weighted_accumulate_f16(ref16, a, 0.37)
    assert np.array_equal(do16.cpu().numpy().view(np.uint16), ref16)
    wdev = _dev(np.array([0.81], dtype=np.float32))
    L.call("vib3_launch_weighted_accumulate_f32_dev_scalar", dacc.data_ptr(), da.data_ptr(),
           wdev.data_ptr(), n, _stream())
    ref = ref.astype(np.float32)
    O.weighted_accumulate_f32(ref, a, 0.81)
    assert np.array_equal(dacc.cpu().numpy(), ref)


# ---------------------------------------------------------------- router

def topk_margin_ok(sel_keys, k):
    s = np.sort(sel_keys)[::-1]
    return s[k - 1] - s[k] > 1e-3


@pytest.mark.parametrize("E,D,k,mode,wdt,xdt,bias", [
    (384, 7168, 8, 1, O.F32, O.BF16, True),    # Kimi-K2.5 / DeepSeek-V3 router
    (8, 4096, 2, 0, O.F32, O.F16, False),      # Mixtral router
    (256, 2048, 8, 1, O.F16, O.F32, False),
    (384, 7168, 8, 0, O.BF16, O.BF16, False),
    (1000, 512, 16, 1, O.F32, O.F32, True),    # not a power of two, k=16
    (5, 64, 5, 0, O.F32, O.F32, False),        # k == E
])
def test_router_topk_ex_parity(E, D, k, mode, wdt, xdt, bias):
    L = _lib()
    _say(f"case: router E={E} D={D} k={k} mode={mode}")
    seed = 0x5EED0002
    w = O.synth_normal_array(seed, 0xF0000000 + E, 0, E * D, 0.01, wdt)
    bvec = O.synth_normal_array(seed, 0xF1000000, 0, E, 0.1, O.F32) if bias else None
    xt, xh = act(D, xdt)
    dw = _dev(w)
    dbias = _dev(bvec) if bias else None
    ids = torch.empty(k, dtype=torch.int16, device="cuda")
    wts = torch.empty(k, dtype=torch.float32, device="cuda")
    scores = torch.empty(E, dtype=torch.float32, device="cuda")
    ws = torch.zeros(L.load().vib3_router_workspace_bytes(E), dtype=torch.uint8, device="cuda")
    for rep in range(2):  # a second call on the same workspace gives the same answer
        L.call("vib3_launch_router_topk_ex", xt.data_ptr(), xdt, dw.data_ptr(), wdt,
               dbias.data_ptr() if bias else None, D, E, k, mode, 2.827, 1, scores.data_ptr(),
               ids.data_ptr(), wts.data_ptr(), ws.data_ptr(), _stream())
        torch.cuda.synchronize()
        r_ids, r_wts, r_scores = O.router(xh, w, wdt, E, D, k, mode, 2.827, True, bvec)
        assert rel_l2(scores.cpu().numpy(), r_scores) <= 1e-5
        got_ids = ids.cpu().numpy().view(np.uint16)
        sig = 1 / (1 + np.exp(-r_scores.astype(np.float64)))
        keys = (sig + (bvec if bias else 0)) if mode == 1 else r_scores
        if k == E or topk_margin_ok(np.asarray(keys), k):
            assert got_ids.tolist() == r_ids.tolist()
            assert np.allclose(wts.cpu().numpy(), r_wts, rtol=1e-5, atol=1e-7)


def test_legacy_router_topk_and_gemv():
    """vib3_launch_router_topk (f32 h, f16 W; sigmoid always normalises) at E=384 — the
    reference kernel's bitonic sort needs a power of two; this one does not."""
    L = _lib()
    _say("case: legacy router")
    E, D, k = 384, 1024, 8
    w = O.synth_normal_array(3, 5, 0, E * D, 0.05, O.F16)
    xt, xh = act(D, O.F32)
    dw = _dev(w)
    scores = torch.empty(E, dtype=torch.float32, device="cuda")
    ids = torch.empty(k, dtype=torch.int16, device="cuda")
    wts = torch.empty(k, dtype=torch.float32, device="cuda")
    L.call("vib3_launch_router_gemv_f32", xt.data_ptr(), dw.data_ptr(), scores.data_ptr(), D, E,
           _stream())
    r_ids, r_wts, r_scores = O.router(xh, w, O.F16, E, D, k, 1, 2.5, True, None)
    assert rel_l2(scores.cpu().numpy(), r_scores) <= 1e-5
    L.call("vib3_launch_router_topk", xt.data_ptr(), dw.data_ptr(), scores.data_ptr(), None,
           ids.data_ptr(), wts.data_ptr(), D, E, k, 1, 2.5, _stream())
    sig = 1 / (1 + np.exp(-r_scores.astype(np.float64)))
    if topk_margin_ok(sig, k):
        assert ids.cpu().numpy().view(np.uint16).tolist() == r_ids.tolist()
        assert np.allclose(wts.cpu().numpy(), r_wts, rtol=1e-5)
    assert float(wts.sum().item()) == pytest.approx(2.5, rel=1e-5)


@pytest.mark.parametrize("E,D", [(8, 4096), (384, 7168)])
def test_router_gemv_f16(E, D):
    """vib3_launch_router_gemv (cuda_ffi.rs:267, kernels.cu:829): f16 h x f16 W -> f32 scores,
    the GEMV of the reference's GPU router branch (kernels.rs:2465); the host then selects."""
    L = _lib()
    _say(f"case: router_gemv E={E} D={D}")
    w = O.synth_normal_array(11, 3, 0, E * D, 0.02, O.F16)
    xt, xh = act(D, O.F16)
    dw = _dev(w)
    scores = torch.full((E,), float("nan"), dtype=torch.float32, device="cuda")
    L.call("vib3_launch_router_gemv", xt.data_ptr(), dw.data_ptr(), scores.data_ptr(), D, E,
           _stream())
    torch.cuda.synchronize()
    _, _, r_scores = O.router(xh, w, O.F16, E, D, 2, 0, 1.0, True, None)
    got = scores.cpu().numpy()
    # f32 sums in another order: |err| <= D * eps * sum|x*w|, far below 1e-5 relative L2
    assert np.isfinite(got).all()
    assert rel_l2(got, r_scores) <= 1e-5
    # the selection the host makes from them (softmax top-2) matches the oracle's
    k = 2
    if topk_margin_ok(r_scores, k):
        assert np.argsort(-got, kind="stable")[:k].tolist() == \
            np.argsort(-r_scores, kind="stable")[:k].tolist()


def test_router_ties_are_stable():
    L = _lib()
    _say("case: router ties")
    E, D, k = 130, 64, 5
    w = np.zeros((E, D), dtype=np.float32)
    w[77] = 0.5
    x = torch.ones(D, dtype=torch.float32, device="cuda")
    dw = _dev(w)
    ids = torch.empty(k, dtype=torch.int16, device="cuda")
    wts = torch.empty(k, dtype=torch.float32, device="cuda")
    ws = torch.zeros(L.load().vib3_router_workspace_bytes(E), dtype=torch.uint8, device="cuda")
    for mode in (0, 1):
        L.call("vib3_launch_router_topk_ex", x.data_ptr(), L.DT_F32, dw.data_ptr(), L.DT_F32, None,
               D, E, k, mode, 1.0, 1, None, ids.data_ptr(), wts.data_ptr(), ws.data_ptr(),
               _stream())
        assert ids.cpu().numpy().view(np.uint16).tolist() == [77, 0, 1, 2, 3]
