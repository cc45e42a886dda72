"""Pins for the CPU oracle (oracle/cpu_ref.c) — CPU only.

Each oracle function is checked against something other than its own formula:
  * the reference's own known-answer tests (tests/integration_test.rs of vib3),
  * brute force in float64 with an independent numpy decode of the page layout,
  * closed forms / invariants (softmax and sigmoid weight sums, bias-only-selects, stable ties),
  * numpy/torch IEEE conversions for f16/bf16 round-to-nearest-even,
so that a swapped nibble, a wrong scale dtype, a dropped -8 offset, a transposed page or a
wrong tie order fails at least one test.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def np_decode_page(page, rows, cols, g, scale_dt):
    """Independent numpy decode of a vib3 INT4 page -> float64 [rows, cols]."""
    pk, ng = (cols + 1) // 2, (cols + g - 1) // g
    data = page[: rows * pk].reshape(rows, pk)
    lo = (data & 0x0F).astype(np.int64) - 8
    hi = (data >> 4).astype(np.int64) - 8
    q = np.empty((rows, pk * 2), dtype=np.int64)
    q[:, 0::2] = lo
    q[:, 1::2] = hi
    q = q[:, :cols]
    sb = page[rows * pk: rows * pk + rows * ng * 2].view(np.uint16).reshape(rows, ng)
    s = O.to_f32(sb, scale_dt).astype(np.float64)
    s = np.where(np.isfinite(s) & (s > 0), s, 0.125)
    return q * np.repeat(s, g, axis=1)[:, :cols]


def rand_page(rng, rows, cols, g, scale_dt, sigma=0.02):
    pk, ng = (cols + 1) // 2, (cols + g - 1) // g
    data = rng.integers(0, 256, rows * pk, dtype=np.uint8)
    s = np.abs(rng.normal(0, sigma, rows * ng)).astype(np.float32)
    if scale_dt == O.BF16:
        sb = (s.view(np.uint32) >> 16).astype(np.uint16)
    else:
        sb = s.astype(np.float16).view(np.uint16)
    sb[sb == 0] = 0x3C00 if scale_dt == O.F16 else 0x3F80
    return np.concatenate([data, sb.view(np.uint8)])


# ---------------------------------------------------------------- reference KATs

def test_kat_int4_lut_matmul_basic():
    """integration_test.rs:1709 — nibbles 0x89,0x88 / 0x98,0x88, BF16 scale 1.0, x=[1,2,3,4]."""
    page = np.array([0x89, 0x88, 0x98, 0x88, 0x80, 0x3F, 0x80, 0x3F], dtype=np.uint8)
    x = O.f16_bits([1.0, 2.0, 3.0, 4.0])
    out = O.to_f32(O.partial_matmul_int4(x, page, 4, 2), O.F16)
    assert out.tolist() == [1.0, 2.0]


def test_kat_int4_lut_matmul_with_scale():
    """integration_test.rs:1788 — 0xAA, BF16 scale 0.5 (0x3f00), x=[3,7] -> 10."""
    page = np.array([0xAA, 0x00, 0x3F], dtype=np.uint8)
    out = O.to_f32(O.partial_matmul_int4(O.f16_bits([3.0, 7.0]), page, 2, 1), O.F16)
    assert out.tolist() == [10.0]


def test_kat_weighted_accumulate():
    """integration_test.rs:420 (restated on the f32 accumulator of kernels.rs:2000)."""
    out = np.array([1, 2, 3, 4], dtype=np.float32)
    O.weighted_accumulate_f32(out, O.f16_bits([10, 20, 30, 40]), 0.5)
    assert out.tolist() == [6.0, 12.0, 18.0, 24.0]


def test_kat_weighted_accumulate_f16():
    """integration_test.rs:420 on its own entry point (weighted_accumulate, kernels.rs:1959):
    f16 accumulator [1, 2, 3, 4] + 0.5 * [10, 20, 30, 40] = [6, 12, 18, 24]; and the f16
    rounding of every sum against numpy's f16 conversion of the exact f64 value."""
    out = O.f16_bits([1, 2, 3, 4])
    O.weighted_accumulate_f16(out, O.f16_bits([10, 20, 30, 40]), 0.5)
    assert O.to_f32(out, O.F16).tolist() == [6.0, 12.0, 18.0, 24.0]
    rng = np.random.default_rng(7)
    o = O.f16_bits(rng.normal(0, 2, 4000))
    e = O.f16_bits(rng.normal(0, 2, 4000))
    ref = (O.to_f32(o, O.F16).astype(np.float32) +
           np.float32(0.37) * O.to_f32(e, O.F16).astype(np.float32)).astype(np.float16)
    O.weighted_accumulate_f16(o, e, 0.37)
    assert np.array_equal(o, ref.view(np.uint16))


def test_kat_run_router_softmax():
    """integration_test.rs:454 — 4 experts, top-2, softmax weights sum to 1; plus closed form."""
    hidden, E = 8, 4
    state = O.to_f32(O.f16_bits([i * 0.1 for i in range(hidden)]), O.F16)
    w = np.zeros((E, hidden), dtype=np.float32)
    for e in range(E):
        w[e, e * 2] = 1.0
    wb = O.f16_bits(w.ravel())
    ids, wts, scores = O.router(state, wb, O.F16, E, hidden, 2, mode=0)
    assert len(ids) == 2 and abs(float(wts.sum()) - 1.0) < 0.01
    assert ids.tolist() == [3, 2]
    d = float(scores[3] - scores[2])
    assert wts[0] == pytest.approx(1.0 / (1.0 + math.exp(-d)), rel=1e-6)


def test_kat_quantize_layout_and_roundtrip():
    """integration_test.rs:2284 (layout size) and :2300 (32x128 gradient, rel err < 0.5)."""
    q = O.quantize_int4(np.array([0.0, 0.5, -0.5, 1.0, -1.0, 0.25, -0.25, 0.0]), 2, 4, 32)
    assert q.size == 2 * 2 + 2 * 1 * 2
    rows, cols = 32, 128
    r = np.arange(rows, dtype=np.float32)[:, None]
    c = np.arange(cols, dtype=np.float32)[None, :]
    w = ((r - 16.0) * (c - 64.0)) / (16.0 * 64.0) * 0.5
    x = (np.arange(cols, dtype=np.float32) / cols) - 0.5
    ref = w.astype(np.float64) @ x.astype(np.float64)
    page = O.quantize_int4(w.ravel(), rows, cols, 32)
    out = O.to_f32(O.partial_matmul_int4(O.f16_bits(x), page, cols, rows), O.F16)
    rel = np.abs(out - ref) / (np.abs(ref) + 1e-6)
    assert rel.max() < 0.5


def test_kat_convert_bf16_fp16_values():
    """integration_test.rs:2420/:2449 value sets through the oracle's RNE converters."""
    for v in [0.0, 1.0, -1.0, 0.5, -0.5, 3.14159, -2.71828, 100.0]:
        b = O.lib().v3o_f32_to_bf16(v)
        f = O.lib().v3o_bf16_to_f32(b)
        assert abs(f - v) < abs(v) * 0.02 + 0.01
    for v in [0.0, 1.0, -1.0, 0.5, -0.5, 0.001]:
        h = O.lib().v3o_f32_to_f16(v)
        assert abs(O.lib().v3o_f16_to_f32(h) - v) < abs(v) * 0.01 + 1e-4


# ---------------------------------------------------------------- conversions vs IEEE libraries

def test_f16_rne_matches_numpy():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 5000), rng.normal(0, 3e4, 5000),
        [65504.0, 65519.0, 65520.0, 1e6, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001, 6.1e-5,
         -0.0, np.inf, -np.inf],
    ]).astype(np.float32)
    ours = O.f16_bits(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    back = np.array([O.lib().v3o_f16_to_f32(int(b)) for b in ours], dtype=np.float32)
    assert np.array_equal(back, ref.view(np.float16).astype(np.float32))


def test_bf16_rne_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    vals = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e-30, 2000),
                           [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.3895e38]]).astype(np.float32)
    ours = np.array([O.lib().v3o_f32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------- brute force

@pytest.mark.parametrize("rows,cols,g,sdt", [(7, 64, 32, O.BF16), (16, 256, 128, O.F16),
                                            (5, 96, 32, O.F16), (3, 7, 32, O.BF16),
                                            (70, 128, 64, O.BF16)])
def test_matmul_int4_bruteforce(rows, cols, g, sdt):
    rng = np.random.default_rng(rows * 1000 + cols)
    page = rand_page(rng, rows, cols, g, sdt)
    x = rng.normal(0, 1, cols).astype(np.float32)
    ref = np_decode_page(page, rows, cols, g, sdt) @ x.astype(np.float64)
    got = O.matmul_int4_acc(x, page, cols, rows, g, sdt)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_matmul_int4_invalid_scale_rule():
    """kernels.rs:2791-2797: zero / negative / NaN / inf scales decode as 1/8."""
    rows, cols, g = 4, 32, 32
    page = np.concatenate([np.full(rows * 16, 0x99, dtype=np.uint8),  # all codes +1
                           np.array([0x0000, 0xBF80, 0x7FC0, 0x7F80], dtype=np.uint16).view(np.uint8)])
    x = np.ones(cols, dtype=np.float32)
    got = O.matmul_int4_acc(x, page, cols, rows, g, O.BF16)
    assert got.tolist() == [4.0] * 4  # 32 * 1 * 0.125


def test_swiglu_bruteforce():
    rng = np.random.default_rng(5)
    rows, cols, g = 33, 128, 32
    up = rand_page(rng, rows, cols, g, O.BF16)
    gate = rand_page(rng, rows, cols, g, O.BF16)
    x = rng.normal(0, 1, cols).astype(np.float32)
    u = np_decode_page(up, rows, cols, g, O.BF16) @ x
    gt = np_decode_page(gate, rows, cols, g, O.BF16) @ x
    ref = gt / (1 + np.exp(-gt)) * u  # SiLU on gate (segment 1), times up (segment 0)
    got = O.swiglu_int4_acc(x, up, gate, cols, rows, g, O.BF16)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    # swapping up and gate must change the answer (pins which operand gets SiLU)
    swapped = O.swiglu_int4_acc(x, gate, up, cols, rows, g, O.BF16)
    assert not np.allclose(swapped, ref, rtol=1e-2)


def test_threads_do_not_change_bits():
    rng = np.random.default_rng(6)
    rows, cols = 300, 512
    page = rand_page(rng, rows, cols, 32, O.BF16)
    x = rng.normal(0, 1, cols).astype(np.float32)
    a = O.matmul_int4_acc(x, page, cols, rows, 32, O.BF16, nthreads=1)
    b = O.matmul_int4_acc(x, page, cols, rows, 32, O.BF16, nthreads=7)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- router invariants

def test_router_sigmoid_bias_selects_only():
    rng = np.random.default_rng(7)
    E, D, k = 384, 64, 8
    x = rng.normal(0, 1, D).astype(np.float32)
    W = rng.normal(0, 0.1, (E, D)).astype(np.float32)
    bias = rng.normal(0, 0.1, E).astype(np.float32)
    ids, wts, scores = O.router(x, W, O.F32, E, D, k, mode=1, scaling=2.827, normalize=True,
                                bias=bias)
    s64 = W.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(scores, s64, rtol=1e-5, atol=1e-5)
    sig = 1 / (1 + np.exp(-scores.astype(np.float64)))
    sel = sig + bias
    order = sorted(range(E), key=lambda e: (-sel[e], e))[:k]
    assert ids.tolist() == order
    ref_w = sig[order] / sig[order].sum() * 2.827
    assert np.allclose(wts, ref_w, rtol=1e-5)
    assert float(wts.sum()) == pytest.approx(2.827, rel=1e-5)
    # without bias the selection follows plain sigmoid order, weights are the same formula
    ids2, _, _ = O.router(x, W, O.F32, E, D, k, mode=1, scaling=2.827, bias=None)
    assert ids2.tolist() == sorted(range(E), key=lambda e: (-sig[e], e))[:k]


def test_router_sigmoid_no_normalize():
    x = np.array([1.0, 0.0], dtype=np.float32)
    W = np.array([[0.0, 0], [1.0, 0], [2.0, 0]], dtype=np.float32)
    ids, wts, _ = O.router(x, W, O.F32, 3, 2, 2, mode=1, scaling=2.0, normalize=False)
    assert ids.tolist() == [2, 1]
    assert np.allclose(wts, 2.0 / (1 + np.exp(-np.array([2.0, 1.0]))), rtol=1e-6)


def test_router_stable_ties():
    x = np.ones(4, dtype=np.float32)
    W = np.zeros((6, 4), dtype=np.float32)
    W[3] = 0.25
    ids, wts, _ = O.router(x, W, O.F32, 6, 4, 3, mode=0)
    assert ids.tolist() == [3, 0, 1]  # ties keep ascending index (stable sort)
    ids, _, _ = O.router(x, W, O.F32, 6, 4, 3, mode=1, scaling=1.0)
    assert ids.tolist() == [3, 0, 1]


def test_router_softmax_equals_full_softmax_renormalised():
    rng = np.random.default_rng(8)
    E, D, k = 8, 4096, 2
    x = rng.normal(0, 1, D).astype(np.float32)
    W = rng.normal(0, 0.02, (E, D)).astype(np.float32)
    ids, wts, scores = O.router(x, W, O.F32, E, D, k, mode=0)
    p = np.exp(scores - scores.max()) / np.exp(scores - scores.max()).sum()
    top = np.argsort(-p, kind="stable")[:k]
    assert ids.tolist() == top.tolist()
    assert np.allclose(wts, p[top] / p[top].sum(), rtol=1e-5)


# ---------------------------------------------------------------- layer composition

@pytest.mark.parametrize("sw", [None, 0.25])
def test_moe_layer_matches_dense_f64(sw):
    """validation.rs:122 forward_moe semantics (dense SwiGLU experts, weighted sum) in f64 on the
    decoded weights, with multi-page experts (rows split over pages); sw: the shared expert's
    sigmoid-gate weight (engine.rs:6418), None for the ungated weight 1.0."""
    rng = np.random.default_rng(9)
    hidden, inter, g, E = 128, 64, 32, 6
    x = rng.normal(0, 1, hidden).astype(np.float32)

    def make_expert(rpp_up, rpp_down):
        mats = {}
        pages = []
        for seg, (rows, cols, rpp) in enumerate([(inter, hidden, rpp_up), (inter, hidden, rpp_up),
                                                 (hidden, inter, rpp_down)]):
            full = rand_page(rng, rows, cols, g, O.BF16, sigma=0.05)
            dense = np_decode_page(full, rows, cols, g, O.BF16)
            mats[seg] = dense
            pk, ng = (cols + 1) // 2, (cols + g - 1) // g
            data = full[: rows * pk].reshape(rows, pk)
            sc = full[rows * pk:].reshape(rows, ng * 2)
            plist = []
            for r0 in range(0, rows, rpp):
                r1 = min(rows, r0 + rpp)
                plist.append(np.concatenate([data[r0:r1].ravel(), sc[r0:r1].ravel()]))
            pages.append(plist)
        return (pages, [rpp_up, rpp_up, rpp_down]), mats

    experts = [make_expert(16, 40) for _ in range(E)]
    shared = make_expert(64, 128)
    ids = np.array([4, 1], dtype=np.uint16)
    wts = np.array([0.7, 0.3], dtype=np.float32)
    shw = None if sw is None else [sw]
    got = O.moe_layer(x, hidden, inter, g, O.BF16, {i: experts[i][0] for i in range(E)}, ids, wts,
                      [shared[0]], faithful=False, shared_weights=shw)
    ref = np.zeros(hidden)
    for e, w in list(zip(ids.tolist(), wts.tolist())) + [(None, 1.0 if sw is None else sw)]:
        m = shared[1] if e is None else experts[e][1]
        up, gate = m[0] @ x, m[1] @ x
        h = gate / (1 + np.exp(-gate)) * up
        ref += w * (m[2] @ h)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 1e-5
    faithful = O.moe_layer(x, hidden, inter, g, O.BF16, {i: experts[i][0] for i in range(E)}, ids,
                           wts, [shared[0]], faithful=True, shared_weights=shw)
    rel_f = np.linalg.norm(faithful - ref) / np.linalg.norm(ref)
    assert 0 < rel_f < 1e-3  # f16 rounding of h and of each down output only


# ---------------------------------------------------------------- MXFP4

def test_e2m1_e8m0_closed_form():
    for code in range(16):
        sign = -1.0 if code & 8 else 1.0
        e, m = (code >> 1) & 3, code & 1
        val = (m * 0.5) if e == 0 else (1 + m * 0.5) * 2.0 ** (e - 1)
        assert O.e2m1(code) == sign * val
    for e in [1, 119, 123, 127, 128, 254]:
        assert O.e8m0(e) == 2.0 ** (e - 127)
    assert O.e8m0(0) == 0.0


def test_matmul_mxfp4_bruteforce():
    rng = np.random.default_rng(10)
    rows, cols = 9, 256
    codes = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = rng.integers(119, 124, rows * cols // 32, dtype=np.uint8)
    x = rng.normal(0, 1, cols).astype(np.float32)
    lut = np.array([O.e2m1(c) for c in range(16)])
    q = np.empty((rows, cols), dtype=np.int64)
    q[:, 0::2] = (codes.reshape(rows, -1) & 15)
    q[:, 1::2] = (codes.reshape(rows, -1) >> 4)
    w = lut[q] * np.repeat(2.0 ** (scales.reshape(rows, -1).astype(np.float64) - 127), 32, axis=1)
    ref = w @ x
    got = O.matmul_mxfp4_acc(x, codes, scales, cols, rows)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


def _mx_dense(page, rows, k):
    """f64 dense matrix of an MXFP4 page (independent of the oracle's C decode)."""
    lut = np.array([(-1.0 if c & 8 else 1.0) * [0, 0.5, 1, 1.5, 2, 3, 4, 6][c & 7]
                    for c in range(16)])
    codes = page[: rows * k // 2].reshape(rows, k // 2)
    sc = page[rows * k // 2: rows * k // 2 + rows * k // 32].reshape(rows, k // 32)
    q = np.empty((rows, k), dtype=np.int64)
    q[:, 0::2] = codes & 15
    q[:, 1::2] = codes >> 4
    return lut[q] * np.repeat(2.0 ** (sc.astype(np.float64) - 127), 32, axis=1)


def test_moe_mxfp4_batched_matches_dense_f64():
    """The per-token MXFP4 composition against an f64 recomputation with the same f16 rounding
    points (h and each expert output); a skipped out-of-range pick contributes nothing."""
    hidden, inter, E, T, k = 128, 96, 6, 3, 3
    pages = [tuple(O.synth_mxfp4_page(5, 3 * e + s, *( (hidden, 0, inter) if s < 2 else (inter, 0, hidden)))
                   for s in range(3)) for e in range(E)]
    rng = np.random.default_rng(4)
    x = O.to_f32(O.synth_normal_array(5, 99, 0, T * hidden, 1.0, O.BF16), O.BF16).reshape(T, hidden)
    ids = np.array([[0, 3, 5], [2, 2, 1], [4, E, 0]], dtype=np.uint16)  # E = out of range
    w = rng.random((T, k)).astype(np.float32)
    got = O.to_f32(O.moe_mxfp4_batched(x, hidden, inter, pages, ids, w).ravel(), O.BF16).reshape(T, hidden)
    ref = np.zeros((T, hidden))
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if e >= E:
                continue
            up = _mx_dense(pages[e][0], inter, hidden) @ x[t]
            gate = _mx_dense(pages[e][1], inter, hidden) @ x[t]
            h = (gate / (1 + np.exp(-gate)) * up).astype(np.float16).astype(np.float64)
            d = (_mx_dense(pages[e][2], hidden, inter) @ h).astype(np.float16).astype(np.float64)
            ref[t] += w[t, j] * d
    # bf16 output rounding (2^-9) dominates; a wrong term, sign or index is far outside it
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-4 * np.abs(ref).max())


def test_synth_mxfp4_page():
    k, rows = 256, 24
    page = O.synth_mxfp4_page(7, 5, k, 0, rows)
    assert np.array_equal(page[: rows * k // 2], O.synth_bytes(7, 10, 0, rows * k // 2))
    sc = page[rows * k // 2:]
    assert sc.size == rows * k // 32 and sc.min() >= 119 and sc.max() <= 123
    assert np.all(np.bincount(sc, minlength=124)[119:] > 0)
    part = O.synth_mxfp4_page(7, 5, k, 8, 4)  # rows 8..11 cut from the same logical matrix
    assert np.array_equal(part[: 4 * k // 2], page[8 * k // 2: 12 * k // 2])
    assert np.array_equal(part[4 * k // 2:], sc[8 * k // 32: 12 * k // 32])


# ---------------------------------------------------------------- synthetic generator

def test_synth_normal_moments_and_scales():
    v = O.synth_normal_array(0x5EED0002, 7, 0, 200000, 1.0, O.F32)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    assert np.abs(v).max() <= 3.47
    page = O.synth_int4_page(0x5EED0002, 3, 256, 32, O.BF16, 0.01, 0, 64)
    sb = page[64 * 128:].view(np.uint16)
    assert np.all((sb & 0x7FFF) != 0) and np.all(sb < 0x8000)
    s = O.to_f32(sb, O.BF16)
    assert 0.004 < s.mean() < 0.012  # E|N(0, 0.01)| = 0.00798
    codes = np.concatenate([page[: 64 * 128] & 15, page[: 64 * 128] >> 4])
    counts = np.bincount(codes, minlength=16)
    assert counts.min() > 0.8 * codes.size / 16


def test_synth_page_is_layout_independent():
    """Rows [a, b) written as one page equal the same rows cut out of the full matrix page."""
    k, g, rows = 256, 32, 40
    full = O.synth_int4_page(1, 9, k, g, O.F16, 0.02, 0, rows)
    part = O.synth_int4_page(1, 9, k, g, O.F16, 0.02, 8, 16)
    pk, ng = k // 2, k // g
    assert np.array_equal(part[: 16 * pk], full[8 * pk: 24 * pk])
    assert np.array_equal(part[16 * pk:], full[rows * pk + 8 * ng * 2: rows * pk + 24 * ng * 2])


# ---------------------------------------------------------------- either side of the MoE

def test_kat_rms_norm():
    """integration_test.rs:701 test_rms_norm: [1,2,3,4], unit weights, eps 1e-6 ->
    x / sqrt(7.5 + eps); and :738 (unit weights) [3,4,0,0] -> [1.2, 1.6, 0, 0]."""
    one = np.full(4, 1.0, np.float16).view(np.uint16)
    y = O.rms_norm_f32(np.array([1, 2, 3, 4], np.float32), one, 1e-6)
    rms = np.sqrt(np.float32(7.5) + np.float32(1e-6))
    assert np.all(np.abs(y - np.array([1, 2, 3, 4]) / rms) < 0.01)
    y = O.rms_norm_f32(np.array([3, 4, 0, 0], np.float32), one, 1e-6)
    assert np.allclose(y, [1.2, 1.6, 0, 0], atol=0.01)


@pytest.mark.parametrize("n,sigma,eps", [(7168, 30.0, 1e-6), (4096, 1.0, 1e-5),
                                         (1000, 1e-4, 1e-6), (300, 1.0, 0.5)])
def test_rms_norm_against_float64(n, sigma, eps):
    """Closed form in float64: y = x / sqrt(mean(x^2) + eps) * w. The tiny-sigma case is
    dominated by eps (a dropped eps or a divide by n - 1 fails it), the weights are not 1 (a
    dropped weight fails), the last case has eps of the order of mean(x^2)."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * sigma).astype(np.float32)
    w = (rng.random(n) + 0.5).astype(np.float16)
    y = O.rms_norm_f32(x, w.view(np.uint16), eps)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + eps) * w.astype(np.float64)
    assert np.max(np.abs(y - ref)) <= 4e-7 * np.max(np.abs(ref))


def test_shared_gate_pieces():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(2048).astype(np.float32)
    w = (rng.standard_normal(2048) * 0.02).astype(np.float16)
    g = O.linear_row_f16(x, w.view(np.uint16))
    assert abs(g - float(np.dot(x.astype(np.float64), w.astype(np.float64)))) < 1e-5
    for v in (-20.0, -1.0, 0.0, 0.5, 30.0):
        assert abs(O.sigmoid(v) - 1 / (1 + np.exp(-v))) < 1e-7
    acc = rng.standard_normal(100).astype(np.float32)
    lo = rng.standard_normal(100).astype(np.float32)
    assert np.array_equal(O.residual_add_f32(acc, lo), acc + lo)

