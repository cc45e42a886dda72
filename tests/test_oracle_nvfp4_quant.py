"""Pins of the oracle's NVFP4 weight quantizers (oracle/cpu_ref.c v3o_quantize_weights_to_nvfp4,
v3o_quantize_half_to_nvfp4, v3o_convert_int4_to_nvfp4, v3o_fp16_to_nvfp4_weight), each against
something other than its own code: a numpy brute force over the E2M1 grid (nearest magnitude,
a value on a midpoint going to the larger one, kernels.rs:4052-4072), numpy's own f16 / bf16
conversions, the dequantization error bound max|w - deq| <= scale (half the widest grid gap,
between 4 and 6), and composition identities between the quantizers. The reference has no test
of these functions. CPU only."""
import numpy as np
import pytest

from oracle import oracle as O

GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float64)


def brute_nearest(a):
    """Index of the nearest grid magnitude to a (>= 0, <= 6), ties to the larger index."""
    d = np.abs(GRID - float(a))
    best = d.min()
    return int(np.nonzero(d == best)[0].max())


def brute_quant(w, rows, cols):
    """Independent restatement: numpy f32 arithmetic and numpy's f16 conversion."""
    w = np.asarray(w, dtype=np.float32).reshape(rows, cols)
    pk, nb = (cols + 1) // 2, (cols + 31) // 32
    data = np.zeros((rows, pk), dtype=np.uint8)
    sc = np.zeros((rows, nb), dtype=np.float16)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        for r in range(rows):
            for b in range(nb):
                blk = w[r, b * 32:min(cols, b * 32 + 32)]
                amax = np.float32(0.0)
                for v in blk:  # f32::max ignores NaN
                    if not np.isnan(v):
                        amax = max(amax, np.float32(abs(v)))
                scale = np.float32(amax / np.float32(6.0)) if amax > 0 else np.float32(1.0)
                sc[r, b] = np.float16(scale)
                for i, v in enumerate(blk):
                    c = b * 32 + i
                    q = np.float32(abs(v)) / scale
                    q = np.float32(6.0) if np.isnan(q) else min(q, np.float32(6.0))
                    nib = brute_nearest(q) | (8 if v < 0 else 0)
                    data[r, c // 2] |= nib if c % 2 == 0 else nib << 4
    return np.concatenate([data.ravel(), sc.view(np.uint8).ravel()])


def dequant(page, rows, cols):
    pk, nb = (cols + 1) // 2, (cols + 31) // 32
    data = page[:rows * pk].reshape(rows, pk)
    sc = page[rows * pk:].view(np.float16).reshape(rows, nb).astype(np.float64)
    out = np.zeros((rows, cols))
    for c in range(cols):
        q = (data[:, c // 2] >> (4 * (c % 2))) & 15
        mag = GRID[q & 7] * np.where(q & 8, -1.0, 1.0)
        out[:, c] = mag * sc[:, c // 32]
    return out


@pytest.mark.parametrize("rows,cols", [(4, 64), (3, 33), (2, 100), (16, 256)])
def test_quantizer_matches_brute_force(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    w[::7] = 0.0
    if cols > 40:
        w[cols:cols + 32] = 0.0  # an all-zero block: scale 1.0, codes 0
    got = O.quantize_weights_to_nvfp4(w, rows, cols)
    assert np.array_equal(got, brute_quant(w, rows, cols))


def test_quantizer_grid_points_and_midpoints():
    """Values on the grid reproduce it; values on the midpoints go up (the reference ladder)."""
    # block max 6 -> scale exactly 1.0
    vals = np.array([6, 0, .5, 1, 1.5, 2, 3, 4, .25, .75, 1.25, 1.75, 2.5, 3.5, 5,
                     -.25, -5, .2499, 4.999, -6, -0.0] + [0] * 11, dtype=np.float32)
    page = O.quantize_weights_to_nvfp4(vals, 1, 32)
    codes = [(page[c // 2] >> (4 * (c % 2))) & 15 for c in range(32)]
    assert codes[:8] == [7, 0, 1, 2, 3, 4, 5, 6]
    assert codes[8:15] == [1, 2, 3, 4, 5, 6, 7]            # midpoints go to the larger value
    assert codes[15:21] == [8 | 1, 8 | 7, 0, 6, 8 | 7, 0]  # -0.0 is not negative
    assert page[16:18].view(np.float16)[0] == np.float16(1.0)


def test_quantizer_round_trip_bound():
    rng = np.random.default_rng(5)
    rows, cols = 32, 512
    w = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32).reshape(rows, cols)
    page = O.quantize_weights_to_nvfp4(w, rows, cols)
    deq = dequant(page, rows, cols)
    sc = page[rows * cols // 2:].view(np.float16).astype(np.float64).reshape(rows, cols // 32)
    bound = np.repeat(sc, 32, axis=1) * (1.0 + 2.0 ** -9)  # half of the 4..6 gap, f16 scale
    assert np.all(np.abs(deq - w) <= bound)
    # the block maximum is represented as +-6 * scale
    for r in range(rows):
        for b in range(cols // 32):
            blk = w[r, b * 32:(b + 1) * 32]
            i = int(np.argmax(np.abs(blk)))
            q = (page[r * cols // 2 + (b * 32 + i) // 2] >> (4 * (i % 2))) & 7
            assert q == 7


def test_quantizer_non_finite():
    w = np.zeros(64, dtype=np.float32)
    w[3], w[5], w[40] = np.inf, 2.0, np.nan
    got = O.quantize_weights_to_nvfp4(w, 1, 64)
    assert np.array_equal(got, brute_quant(w, 1, 64))
    sc = got[32:].view(np.float16)
    assert np.isinf(sc[0]) and sc[1] == np.float16(1.0)  # NaN is ignored by the block max


@pytest.mark.parametrize("dt", [O.F16, O.BF16])
def test_half_quantizers_widen_then_quantize(dt):
    rng = np.random.default_rng(9)
    rows, cols = 8, 96
    f = (rng.standard_normal(rows * cols) * 0.03).astype(np.float32)
    if dt == O.F16:
        bits = f.astype(np.float16).view(np.uint16)
        wide = bits.view(np.float16).astype(np.float32)
    else:
        bits = (f.view(np.uint32) >> 16).astype(np.uint16)  # truncation: any bf16 pattern
        wide = (bits.astype(np.uint32) << 16).view(np.float32)
    got = O.quantize_half_to_nvfp4(bits, dt, rows, cols)
    assert np.array_equal(got, brute_quant(wide, rows, cols))


def int4_page(rng, rows, cols, g):
    pk, ng = (cols + 1) // 2, (cols + g - 1) // g
    data = rng.integers(0, 256, rows * pk, dtype=np.uint8)
    if cols % 2:
        data.reshape(rows, pk)[:, -1] &= 0x0F
    sc = (np.abs(rng.standard_normal(rows * ng)) * 0.01 + 1e-4).astype(np.float32)
    scb = (sc.view(np.uint32) >> 16).astype(np.uint16)
    return np.concatenate([data, scb.view(np.uint8)])


def int4_dequant(page, rows, cols, g, length=None):
    """numpy restatement of the INT4 dequantization with BF16 scales, and the reference's
    bounds rule (a scale whose bytes lie past `length` reads as 1.0)."""
    length = page.size if length is None else length
    pk, ng = (cols + 1) // 2, (cols + g - 1) // g
    out = np.zeros((rows, cols), dtype=np.float32)
    for r in range(rows):
        for c in range(cols):
            q = (page[r * pk + c // 2] >> (4 * (c % 2))) & 15
            off = rows * pk + (r * ng + c // g) * 2
            if off + 1 < length:
                s = np.array([(int(page[off]) | (int(page[off + 1]) << 8)) << 16], dtype=np.uint32).view(np.float32)[0]
            else:
                s = np.float32(1.0)
            out[r, c] = np.float32(int(q) - 8) * s
    return out


@pytest.mark.parametrize("rows,cols,g", [(4, 128, 32), (3, 100, 32), (2, 256, 128), (5, 33, 32)])
def test_convert_int4_is_dequantize_then_quantize(rows, cols, g):
    rng = np.random.default_rng(rows + cols + g)
    page = int4_page(rng, rows, cols, g)
    got = O.convert_int4_to_nvfp4(page, rows, cols, g)
    want = brute_quant(int4_dequant(page, rows, cols, g), rows, cols)
    assert np.array_equal(got, want)
    # and equal to the oracle's own INT4 dequantizer composed with its NVFP4 quantizer
    deq = O.dequantize_int4(page, rows, cols, g, O.BF16)
    assert np.array_equal(got, O.quantize_weights_to_nvfp4(deq, rows, cols))


def test_convert_int4_bounds_rule():
    """A page cut short: scales past the end read as 1.0 (kernels.rs:3995-4003)."""
    rows, cols, g = 2, 64, 32
    page = int4_page(np.random.default_rng(3), rows, cols, g)[:-2]
    got = O.convert_int4_to_nvfp4(page, rows, cols, g)
    assert np.array_equal(got, brute_quant(int4_dequant(page, rows, cols, g), rows, cols))


def brute_e8m0(amax):
    """round(log2 amax) - 2 + 127 (round half up in the log domain), clamped."""
    if amax <= 0:
        return 0
    return int(np.clip(np.floor(np.log2(np.float64(amax)) + 0.5) - 2 + 127, 0, 254))


def test_fp16_to_nvfp4_weight_brute_force():
    """kernels.cu:6017: each group's E8M0 exponent is the rounded log2 of its max minus 2, and
    every code is the nearest E2M1 value of v / 2^(e-127) (ties to the even code); layout
    split-half within each 32-value group, scale stored as bf16 bits e << 7."""
    rng = np.random.default_rng(11)
    m, k = 6, 128
    w = (rng.standard_normal(m * k) * 0.02).astype(np.float16)
    w[5 * k:5 * k + 32] = 0
    data, sc = O.fp16_to_nvfp4_weight(w.view(np.uint16), m, k)
    wf = w.astype(np.float64).reshape(m, k)
    for r in range(m):
        for g in range(k // 32):
            blk = wf[r, g * 32:(g + 1) * 32]
            e = brute_e8m0(np.abs(blk).max())
            assert sc[r * (k // 32) + g] == e << 7
            step = 2.0 ** (127 - e) if np.abs(blk).max() > 0 else 0.0
            for j in range(32):
                byte = data[r * k // 2 + g * 16 + (j % 16)]
                q = (byte >> (4 * (j >= 16))) & 15
                a = min(abs(blk[j] * step), 6.0)
                d = np.abs(GRID - a)
                cands = np.nonzero(d == d.min())[0]
                want = cands[0] if len(cands) == 1 else [c for c in cands if c % 2 == 0][0]
                assert q & 7 == want
                if want:
                    assert bool(q & 8) == (blk[j] < 0)


def test_fp16_to_nvfp4_weight_is_the_activation_quantizer_per_row():
    rng = np.random.default_rng(12)
    m, k = 4, 256
    w = (rng.standard_normal(m * k) * 0.5).astype(np.float16)
    data, sc = O.fp16_to_nvfp4_weight(w.view(np.uint16), m, k)
    for r in range(m):
        c, e = O.fp4_quantize_act(w[r * k:(r + 1) * k].astype(np.float32))
        assert np.array_equal(data[r * k // 2:(r + 1) * k // 2], c)
        assert np.array_equal(sc[r * k // 32:(r + 1) * k // 32], e.astype(np.uint16) << 7)
