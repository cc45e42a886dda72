"""Pins of the oracle's per-page NVFP4 GEMVs (oracle/cpu_ref.c v3o_nvfp4_page_matvec,
v3o_nvfp4_page_swiglu, v3o_nvfp4_seq_matvec_f64) against pieces pinned elsewhere and an
independent numpy decode: the tiled layout equals v3o_nvfp4_matvec (pinned in
test_oracle_fp4.py), the row-major split-half and sequential layouts equal it after the
reference's own repacks (v3o_fp4_to_tiled, v3o_fp4_split_half), a full bf16 scale with a zero
mantissa equals its E8M0 reading, and a float64 numpy decode gives the same numbers. CPU only."""
import numpy as np
import pytest

from oracle import oracle as O

E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])


def rand_act(rng, k):
    x = (rng.standard_normal(k) * rng.uniform(0.1, 4.0)).astype(np.float32)
    return O.fp4_quantize_act(x)


def rand_weights(rng, m, k, e8m0=True):
    data = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
    if e8m0:
        sc = (rng.integers(118, 126, m * k // 32).astype(np.uint16) << 7)
    else:
        sc = (np.abs(rng.standard_normal(m * k // 32)) * 0.01).astype(np.float32)
        sc = (sc.view(np.uint32) >> 16).astype(np.uint16)
    return data, sc


def decode_split(codes, k):
    """numpy decode of split-half codes (byte j of a group: value j low, value j + 16 high)."""
    c = codes.reshape(-1, 16)
    out = np.zeros((c.shape[0], 32))
    out[:, :16] = E2M1[c & 15]
    out[:, 16:] = E2M1[c >> 4]
    return out.ravel()[:k]


def decode_seq(row_bytes, k):
    out = np.zeros(k)
    out[0::2] = E2M1[row_bytes & 15][: (k + 1) // 2]
    out[1::2] = E2M1[row_bytes >> 4][: k // 2]
    return out


M, K = 32, 256


def test_tiled_layout_is_the_pinned_matvec():
    rng = np.random.default_rng(1)
    ac, asc = rand_act(rng, K)
    d, s = rand_weights(rng, M, K)
    assert np.array_equal(O.nvfp4_page_matvec(ac, asc, d, s, M, K, 1),
                          O.nvfp4_matvec(ac, asc, d, s, M, K))


def test_row_major_layouts_after_the_reference_repacks():
    rng = np.random.default_rng(2)
    ac, asc = rand_act(rng, K)
    seq, s = rand_weights(rng, M, K)
    split = O.fp4_split_half(seq)          # kernels.cu:4132 repack_weights_inplace
    tiled = O.fp4_to_tiled(split, M, K)     # kernels.cu:4190 repack_row_to_tiled
    want = O.nvfp4_matvec(ac, asc, tiled, s, M, K)
    assert np.array_equal(O.nvfp4_page_matvec(ac, asc, split, s, M, K, 0), want)
    assert np.array_equal(O.nvfp4_page_matvec(ac, asc, seq, s, M, K, 2), want)


@pytest.mark.parametrize("e8m0", [True, False])
def test_full_bf16_scales_against_numpy(e8m0):
    rng = np.random.default_rng(3 + e8m0)
    ac, asc = rand_act(rng, K)
    d, s = rand_weights(rng, M, K, e8m0=e8m0)
    a = decode_split(ac, K) * np.repeat(2.0 ** (asc.astype(np.float64) - 127), 32)
    sw = (s.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(M, K // 32)
    want = np.array([np.sum(decode_split(d[r * K // 2:(r + 1) * K // 2], K) *
                            np.repeat(sw[r], 32) * a) for r in range(M)], dtype=np.float32)
    got = O.nvfp4_page_matvec(ac, asc, d, s, M, K, 0, full=True)
    assert np.array_equal(got, want)
    if e8m0:  # mantissa zero: the full value is the E8M0 power of two
        assert np.array_equal(got, O.nvfp4_page_matvec(ac, asc, d, s, M, K, 0, full=False))


def test_swiglu_of_page_gemvs():
    rng = np.random.default_rng(5)
    ac, asc = rand_act(rng, K)
    up, us = rand_weights(rng, M, K)
    gt, gs = rand_weights(rng, M, K)
    u = O.nvfp4_page_matvec(ac, asc, up, us, M, K, 0).astype(np.float64)
    g = O.nvfp4_page_matvec(ac, asc, gt, gs, M, K, 0).astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    got = O.nvfp4_page_swiglu(ac, asc, up, us, gt, gs, M, K, 0)
    assert np.allclose(got, want, rtol=3e-7, atol=1e-30)


def test_seq_matvec_f64_against_numpy():
    rng = np.random.default_rng(6)
    x = rng.standard_normal(K).astype(np.float32)
    d, s = rand_weights(rng, M, K, e8m0=False)
    sw = (s.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(M, K // 32)
    want = np.array([np.sum(decode_seq(d[r * K // 2:(r + 1) * K // 2], K) *
                            np.repeat(sw[r], 32) * x.astype(np.float64)) for r in range(M)])
    got = O.nvfp4_seq_matvec_f64(x, d, s, M, K)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-300)
