"""Pins of the oracle's NVFP4 fused-MoE restatement (oracle/cpu_ref.c v3o_fp4_*, v3o_nvfp4_*,
v3o_moe_experts_fused), each against something other than its own formula: the reference's
own known answers (the MMA self-test pattern and the activation quantizer example,
cuda/src/kernels.cu:2780-2800), brute force over the E2M1 grid, float64 closed forms computed
here from an independent decode, and libm's exp. CPU only."""
import math

import numpy as np
import pytest

from oracle import oracle as O

GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def ulp_dist(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def test_exp_within_two_ulp_of_libm():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-87.0, 88.7, 20000), rng.uniform(-1, 1, 5000),
                         [0.0, -0.0, 1.0, -1.0, 88.72, -87.33, 1e-8, -1e-8]]).astype(np.float32)
    got = np.array([O.exp_cw(float(x)) for x in xs], dtype=np.float32)
    ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert ulp_dist(got, ref).max() <= 2
    assert O.exp_cw(100.0) == math.inf and O.exp_cw(-200.0) == 0.0
    assert math.isnan(O.exp_cw(float("nan")))
    # subnormal results: within 2 units of the smallest subnormal
    sub = np.float32(-100.0)
    assert abs(O.exp_cw(float(sub)) - math.exp(float(sub))) <= 2 * 2.0 ** -149


def brute_e2m1(v):
    """Nearest E2M1 magnitude, ties to the even code, saturating at 6; sign of v."""
    a = min(abs(v), 6.0)
    d = np.abs(GRID - a)
    best = np.flatnonzero(d == d.min())
    c = int(best[0]) if len(best) == 1 else int([b for b in best if b % 2 == 0][0])
    return (8 if math.copysign(1.0, v) < 0 else 0) | c


def test_e2m1_round_to_nearest_even_brute_force():
    vals = list(np.arange(-8, 8.0001, 1 / 64)) + list(np.random.default_rng(1).normal(0, 3, 3000))
    vals += [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -5.0, 1e9, -1e9, -0.0]
    for v in vals:
        assert O.e2m1_rne(float(np.float32(v))) == brute_e2m1(float(np.float32(v))), v


def test_e8m0_of_amax_is_round_log2_minus_2():
    """compute_e8m0 (kernels.cu:2759): round(log2 amax) - 2 + 127, clamped; the reference's
    comment gives amax = 1.0 -> 125 (kernels.cu:2792-2794)."""
    assert O.fp4_e8m0_of_amax(1.0) == 125
    assert O.fp4_e8m0_of_amax(0.0) == 0 and O.fp4_e8m0_of_amax(-1.0) == 0
    rng = np.random.default_rng(2)
    a = (rng.uniform(1, 2, 5000) * 2.0 ** rng.integers(-120, 120, 5000)).astype(np.float32)
    for v in a:
        r = int(np.rint(np.log2(np.float64(v)))) - 2 + 127
        assert O.fp4_e8m0_of_amax(float(v)) == min(max(r, 0), 254)
    # the rounding boundary sqrt 2: just below rounds down, just above up
    below = np.float32(1.41421353816986083984375)  # float below sqrt 2
    assert O.fp4_e8m0_of_amax(float(below)) == 125
    assert O.fp4_e8m0_of_amax(float(np.nextafter(below, np.float32(2)))) == 126


def split_decode(codes, k):
    """Element values of a split-half code vector (independent decode)."""
    codes = np.asarray(codes, np.uint8)
    out = np.empty(k, np.uint8)
    for g in range(k // 32):
        blk = codes[g * 16:(g + 1) * 16]
        out[g * 32:g * 32 + 16] = blk & 15
        out[g * 32 + 16:g * 32 + 32] = blk >> 4
    return out


def e2m1_val(c):
    c = np.asarray(c, np.int64)
    return np.where(c & 8, -1.0, 1.0) * GRID[c & 7]


def test_quantize_act_reference_example_and_bounds():
    """kernels.cu:2786-2797: an activation of all 1.0 gets scale 125 (0.25) and is stored as
    FP4 4.0 = 0b0110 in both nibbles (0x66). Random inputs: every element dequantizes to the
    nearest grid value of v / 2^(e-127), and e is the group's E8M0."""
    codes, sc = O.fp4_quantize_act(np.ones(64, np.float32))
    assert codes.tolist() == [0x66] * 32 and sc.tolist() == [125, 125]
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, 4096).astype(np.float32)
    x[64:96] = 0.0                       # an all-zero group: scale 0, codes 0
    x[128:160] *= np.float32(1e-30)       # tiny values
    codes, sc = O.fp4_quantize_act(x)
    elems = split_decode(codes, x.size)
    for g in range(x.size // 32):
        v = x[g * 32:(g + 1) * 32].astype(np.float64)
        amax = np.abs(v).max()
        e = 0 if amax == 0 else min(max(int(np.rint(np.log2(amax))) - 2 + 127, 0), 254)
        assert sc[g] == e
        inv = 0.0 if amax == 0 else 2.0 ** (127 - e)
        want = [brute_e2m1(float(np.float32(t * inv))) for t in v]
        assert elems[g * 32:(g + 1) * 32].tolist() == want
    assert sc[2] == 0 and not codes[32:48].any()


def tiled_decode(data, m, k):
    """Codes [m][k] of a tiled split-half matrix, decoded here with numpy."""
    nkt = k // 64
    t = np.asarray(data, np.uint8).reshape(m // 16, nkt, 16, 2, 16)  # rb, tile, row, grp, byte
    lo, hi = t & 15, t >> 4
    grp = np.concatenate([lo, hi], axis=-1)                          # ..., grp, 32 values
    return grp.transpose(0, 2, 1, 3, 4).reshape(m, k)


def dense_matvec(act_codes, act_sc, data, scales, m, k):
    w = e2m1_val(tiled_decode(data, m, k)) * \
        np.repeat(2.0 ** (((np.asarray(scales, np.int64) >> 7) & 0xFF) - 127), 32, axis=1)
    a = e2m1_val(split_decode(act_codes, k)) * np.repeat(2.0 ** (act_sc.astype(np.int64) - 127), 32)
    return (w @ a).astype(np.float32)


def random_page(rng, m, k, exp_lo=119, exp_hi=123):
    data = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
    ew = rng.integers(exp_lo, exp_hi + 1, (m, k // 32))
    scales = ((ew << 7) | rng.integers(0, 128, (m, k // 32))).astype(np.uint16)  # bf16 bits
    return data, scales


def test_matvec_selftest_pattern_and_dense_f64():
    """kernels.cu:2780-2787: weights all 1.0 (code 2, bytes 0x22) times activations 1.0 with
    both scales E8M0 127 over K = 64 give 64.0. Random tiles: the exact f64 matvec of an
    independent numpy decode (bf16 scale mantissas are ignored: only the exponent byte counts)."""
    out = O.nvfp4_matvec(np.full(32, 0x22, np.uint8), np.full(2, 127, np.uint8),
                         np.full(16 * 32, 0x22, np.uint8), np.full((16, 2), 0x3F80, np.uint16), 16, 64)
    assert out.tolist() == [64.0] * 16
    rng = np.random.default_rng(4)
    m, k = 64, 512
    data, scales = random_page(rng, m, k)
    x = rng.normal(0, 1, k).astype(np.float32)
    ac, asc = O.fp4_quantize_act(x)
    got = O.nvfp4_matvec(ac, asc, data, scales, m, k)
    assert np.array_equal(got, dense_matvec(ac, asc, data, scales, m, k))


def test_moe_fused_composition_f64():
    """Two experts through up/gate -> SwiGLU -> FP4 h -> down -> out += w * d, against a numpy
    float64 composition with libm's exp (rel-L2 1e-3: the exps differ by an ulp, which can move
    an h element across an FP4 rounding point) and out accumulated, not overwritten."""
    rng = np.random.default_rng(5)
    k_in, m_mid, m_out = 256, 128, 64
    experts, wts = [], np.array([0.7, -1.3], np.float32)
    for _ in range(2):
        experts.append((random_page(rng, m_mid, k_in, 120, 122),
                        random_page(rng, m_mid, k_in, 120, 122),
                        random_page(rng, m_out, m_mid, 120, 122)))
    x = rng.normal(0, 1, k_in).astype(np.float32)
    ac, asc = O.fp4_quantize_act(x)
    out = rng.normal(0, 1, m_out).astype(np.float32)
    base = out.copy()
    O.moe_experts_fused(ac, asc, experts, wts, k_in, m_mid, m_out, out)
    ref = base.astype(np.float64)
    for (up, gate, down), w in zip(experts, wts):
        u = dense_matvec(ac, asc, *up, m_mid, k_in).astype(np.float64)
        g = dense_matvec(ac, asc, *gate, m_mid, k_in).astype(np.float64)
        h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
        hc, hs = O.fp4_quantize_act(h)
        ref += float(w) * dense_matvec(hc, hs, *down, m_out, m_mid)
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref - base)
    assert rel <= 1e-3


def test_repack_split_half_and_tiled_layouts():
    """kernels.cu:4125-4131: after the in-place repack, byte j of each 16-byte block holds
    element j (low) and element j + 16 (high) of the 32 sequential elements; row -> tiled
    places row r's 32 bytes of k-tile t at (r/16 * nkt + t) * 512 + (r%16) * 32."""
    rng = np.random.default_rng(6)
    seq = rng.integers(0, 256, 4096, dtype=np.uint8)
    elems = np.stack([seq & 15, seq >> 4], axis=1).reshape(-1)  # sequential nibble order
    split = O.fp4_split_half(seq)
    assert np.array_equal(split_decode(split, elems.size), elems)
    part = O.fp4_split_half(seq[:40])  # a partial last block is left as it is
    assert np.array_equal(part[32:], seq[32:40])
    m, k = 48, 256
    row = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
    tiled = O.fp4_to_tiled(row, m, k)
    nkt = k // 64
    for r in range(m):
        for t in range(nkt):
            off = (r // 16 * nkt + t) * 512 + (r % 16) * 32
            assert np.array_equal(tiled[off:off + 32], row[r * k // 2 + t * 32: r * k // 2 + t * 32 + 32])


@pytest.mark.parametrize("k,sigma,eps", [(7168, 20.0, 1e-6), (3072, 1.0, 1e-5), (96, 1e-4, 1e-6)])
def test_fp4_norm_inverse_rms_closed_form(k, sigma, eps):
    """The fused norm's inverse RMS (kernels.cu:6610-6645 order) within 2 ulp of the float64
    closed form 1 / sqrt(mean(x^2) + eps) at residual-stream, unit and eps-dominated
    magnitudes (a dropped eps, a divide by k - 1 or a missing square fails it)."""
    rng = np.random.default_rng(k)
    x = rng.normal(0, sigma, k).astype(np.float32)
    got = np.float32(O.fp4_norm_inv(x, eps))
    want = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)
    assert abs(float(got) - want) <= 2 * float(np.spacing(np.float32(want)))


def test_fused_rms_norm_quantize_known_answer_and_composition():
    """All-ones activation and weights: y = 1/sqrt(1 + eps) ~ 1, so every group gets the
    reference quantizer's all-1.0 answer (scale byte 125, codes 0x66, kernels.cu:2786-2797);
    and in general the fused call equals the norm followed by the standalone quantizer, with
    the f16 output the round-to-nearest-even of the normalised values."""
    k = 256
    codes, sc, h = O.fused_rms_norm_quantize_fp4(np.ones(k, np.float32),
                                                 np.full(k, 0x3C00, np.uint16), 1e-6, f16_out=True)
    assert codes.tolist() == [0x66] * (k // 2) and sc.tolist() == [125] * (k // 32)
    assert np.all(h == np.float16(1.0 / np.sqrt(1 + 1e-6)).view(np.uint16))
    rng = np.random.default_rng(5)
    x = rng.normal(0, 7, 2048).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(2048)).astype(np.float16)
    inv = np.float32(O.fp4_norm_inv(x, 1e-6))
    y = (x * inv).astype(np.float32) * w.astype(np.float32)
    c2, s2 = O.fp4_quantize_act(y.astype(np.float32))
    c1, s1, h1 = O.fused_rms_norm_quantize_fp4(x, w.view(np.uint16), 1e-6, f16_out=True)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)
    assert np.array_equal(h1, y.astype(np.float16).view(np.uint16))


def test_exact_sums_stay_within_the_f32_accumulation_bound():
    """The reference's MMA kernels accumulate each row's 64-value tile products in f32 in
    tile order (kernels.cu:3276-3385, :4544-4700); this build and its oracle sum exactly and
    round once. The two differ by at most the f32 accumulation bound n * 2^-24 * sum |tile|,
    so any drift from the reference's numbers is bounded (observed: ~1e-7 relative)."""
    rng = np.random.default_rng(17)
    m, k = 64, 7168
    x = rng.normal(0, 2, k).astype(np.float32)
    codes, sc = O.fp4_quantize_act(x)
    data = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
    ws = ((rng.integers(119, 124, (m, k // 32)) << 7)).astype(np.uint16)
    exact = O.nvfp4_page_matvec(codes, sc, data, ws, m, k, 0).astype(np.float64)
    g = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])
    a = np.concatenate([np.concatenate([g[c & 15] for c in codes.reshape(-1, 16)[i:i + 1]] +
                                       [g[c >> 4] for c in codes.reshape(-1, 16)[i:i + 1]])
                        for i in range(k // 32)])
    a = a * np.repeat(2.0 ** (sc.astype(np.float64) - 127), 32)
    worst = 0.0
    for r in range(m):
        row = data[r * k // 2:(r + 1) * k // 2].reshape(-1, 16)
        w = np.concatenate([np.concatenate([g[b & 15], g[b >> 4]]) for b in row])
        w = w * np.repeat(2.0 ** (((ws[r].astype(np.int64) >> 7) & 0xFF) - 127), 32)
        tiles = (w * a).reshape(-1, 64).sum(1)           # each tile's sum: exact in f64
        acc = np.float32(0.0)
        for t in tiles:                                   # f32 accumulation in tile order
            acc = np.float32(acc + np.float32(t))
        bound = len(tiles) * 2.0 ** -24 * np.abs(tiles).sum() + 2.0 ** -24 * abs(exact[r])
        assert abs(float(acc) - exact[r]) <= bound
        worst = max(worst, abs(float(acc) - exact[r]) / max(np.abs(tiles).sum(), 1e-30))
    assert worst < 1e-5
