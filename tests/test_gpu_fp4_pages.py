"""GPU parity of the reference's per-page NVFP4 launchers (fp4_pages.hip), the NVFP4 weight
quantizer, expert_batched, and the fused path's buffer rules (lazy allocation, caller
workspaces on concurrent streams), through the C ABI against the CPU oracle.

Bars: the block-scaled kernels are bit-exact (exact group sums, one rounding; SwiGLU with the
oracle's exp). The scalar kernels accumulate in f32 in an order of their own (as the
reference's warp reductions do): within 1e-6 relative L2 of the oracle's f64 sums, f16 outputs
within one f16 ulp of the f64 value rounded."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _st():
    return torch.cuda.current_stream().cuda_stream


def dev(a, dt=np.uint8):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dt).view(np.uint8)).cuda()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def rand_codes_scales(rng, m, k, e8m0=True):
    data = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
    ew = rng.integers(119, 124, (m, k // 32))
    mant = 0 if e8m0 else rng.integers(0, 128, (m, k // 32))
    return data, ((ew << 7) | mant).astype(np.uint16)


def quantized_act(rng, k, scale=1.0):
    x = (rng.standard_normal(k) * scale).astype(np.float32)
    codes, sc = O.fp4_quantize_act(x)
    return x, codes, sc


def test_fp16_to_nvfp4_weight_bit_exact():
    from vib3_amd import _lib
    _say("case: fp16_to_nvfp4_weight")
    rng = np.random.default_rng(3)
    m, k = 96, 7168
    w = (rng.standard_normal(m * k) * 0.02).astype(np.float16)
    w[:32] = 0
    din = dev(w.view(np.uint16), np.uint16)
    data = torch.zeros(m * k // 2, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(m * k // 32, dtype=torch.int16, device="cuda")
    _lib.call("vib3_launch_fp16_to_nvfp4_weight", din.data_ptr(), data.data_ptr(), sc.data_ptr(),
              m, k, _st())
    torch.cuda.synchronize()
    rd, rs = O.fp16_to_nvfp4_weight(w.view(np.uint16), m, k)
    assert np.array_equal(data.cpu().numpy(), rd)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), rs)


class PagedExpert:
    """One NVFP4 expert cut into pages of `rpp` rows per matrix (row-major split-half data, then
    the page's scales), as the converter's 2 MiB pages hold them (convert.rs:1853-1865)."""

    def __init__(self, rng, k_in, m_mid, m_out, rpp_gu, rpp_dn):
        self.k_in, self.m_mid, self.m_out = k_in, m_mid, m_out
        self.mats = []  # per matrix: list of (row_start, rows, host data, host scales, dev page)
        for rows, k, rpp in ((m_mid, k_in, rpp_gu), (m_mid, k_in, rpp_gu), (m_out, m_mid, rpp_dn)):
            pages = []
            for r0 in range(0, rows, rpp):
                n = min(rpp, rows - r0)
                d, s = rand_codes_scales(rng, n, k)
                page = dev(np.concatenate([d, s.view(np.uint8).ravel()]))
                pages.append((r0, n, d, s, page))
            self.mats.append(pages)


def test_execute_expert_nvfp4_over_pages_bit_exact():
    """engine.rs:6060-6226 for an NVFP4 expert over several pages per matrix, Kimi shape
    (hidden 7168, expert inter 2048; the converter's 520 / 1820-row pages): per up/gate page
    pair fused_swiglu_mma_nvfp4_preq into h[row_start..], h quantized with
    quantize_activation_fp4, then per down page gemv_mma_nvfp4_preq into d[row_start..]."""
    from vib3_amd import kernels as K
    _say("case: execute_expert nvfp4 pages kimi")
    rng = np.random.default_rng(11)
    ex = PagedExpert(rng, 7168, 2048, 7168, 520, 1820)
    x, codes, sc = quantized_act(rng, 7168, 2.0)
    a, asc = dev(codes), dev(sc)
    h = torch.zeros(2048, dtype=torch.float32, device="cuda")
    for (r0, n, ud, us, up), (_, _, gd, gs, gp) in zip(ex.mats[0], ex.mats[1]):
        K.fused_swiglu_mma_nvfp4_preq(a, asc, up, gp, h[r0:], 7168, n)
    hc = torch.zeros(2048 // 2, dtype=torch.uint8, device="cuda")
    hs = torch.zeros(2048 // 32, dtype=torch.uint8, device="cuda")
    K.quantize_activation_fp4(h, hc, hs, 2048)
    d = torch.zeros(7168, dtype=torch.float32, device="cuda")
    for (r0, n, dd, ds, dp) in ex.mats[2]:
        K.gemv_mma_nvfp4_preq(hc, hs, dp, d[r0:], 2048, n)
    torch.cuda.synchronize()
    ref_h = np.concatenate([O.nvfp4_page_swiglu(codes, sc, ud, us, gd, gs, n, 7168, 0)
                            for (_, n, ud, us, _), (_, _, gd, gs, _) in zip(ex.mats[0], ex.mats[1])])
    assert np.array_equal(h.cpu().numpy(), ref_h)
    rhc, rhs = O.fp4_quantize_act(ref_h)
    ref_d = np.concatenate([O.nvfp4_page_matvec(rhc, rhs, dd, ds, n, 2048, 0)
                            for (_, n, dd, ds, _) in ex.mats[2]])
    assert np.array_equal(d.cpu().numpy(), ref_d)


@pytest.mark.parametrize("entry,lay,full", [
    ("vib3_launch_gemv_mma_nvfp4_preq", 0, False),
    ("vib3_launch_gemv_mma_nvfp4_preq_fast", 0, False),
    ("vib3_launch_gemv_mma_nvfp4_tiled", 1, False),
    ("vib3_launch_gemv_scalar_nvfp4", 0, True),
])
def test_block_scaled_gemv_bit_exact(entry, lay, full):
    from vib3_amd import _lib
    _say(f"case: {entry}")
    rng = np.random.default_rng(21 + lay)
    m, k = 400, 7168 if lay != 1 else 2048
    if lay == 1:
        m = 512
    x, codes, sc = quantized_act(rng, k)
    data, s = rand_codes_scales(rng, m, k, e8m0=not full)
    page = dev(np.concatenate([data, s.view(np.uint8).ravel()]))
    out = torch.full((m,), float("nan"), dtype=torch.float32, device="cuda")
    a, asc = dev(codes), dev(sc)  # (kept alive until the kernel has run)
    _lib.call(entry, a.data_ptr(), asc.data_ptr(), page.data_ptr(),
              page.data_ptr() + data.size, out.data_ptr(), k, m, _st())
    torch.cuda.synchronize()
    want = O.nvfp4_page_matvec(codes, sc, data, s, m, k, lay, full)
    assert np.array_equal(out.cpu().numpy(), want)


def test_mma_gemv_f32_input_bit_exact():
    """vib3_launch_gemv_mma_nvfp4 / _fused_swiglu_mma_nvfp4 (kernels.cu:3676, :3807): the f32
    input is quantized in the kernel with the activation quantizer's rule; sequential codes."""
    from vib3_amd import _lib
    _say("case: gemv_mma_nvfp4 f32 input")
    rng = np.random.default_rng(31)
    m, k = 300, 4096
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    codes, sc = O.fp4_quantize_act(x)
    ud, us = rand_codes_scales(rng, m, k)
    gd, gs = rand_codes_scales(rng, m, k)
    up = dev(np.concatenate([ud, us.view(np.uint8).ravel()]))
    gp = dev(np.concatenate([gd, gs.view(np.uint8).ravel()]))
    xd = torch.from_numpy(x).cuda()
    out = torch.zeros(m, dtype=torch.float32, device="cuda")
    _lib.call("vib3_launch_gemv_mma_nvfp4", xd.data_ptr(), up.data_ptr(), up.data_ptr() + ud.size,
              out.data_ptr(), k, m, _st())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.nvfp4_page_matvec(codes, sc, ud, us, m, k, 2))
    _lib.call("vib3_launch_fused_swiglu_mma_nvfp4", xd.data_ptr(), up.data_ptr(),
              up.data_ptr() + ud.size, gp.data_ptr(), gp.data_ptr() + gd.size, out.data_ptr(), k,
              m, _st())
    torch.cuda.synchronize()
    seq_split = [O.fp4_split_half(v) for v in (ud, gd)]  # the same numbers in layout 0
    want = O.nvfp4_page_swiglu(codes, sc, seq_split[0], us, seq_split[1], gs, m, k, 0)
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("entry,in16,out16,ns", [
    ("vib3_launch_partial_matmul_nvfp4", False, True, 1),
    ("vib3_launch_partial_matmul_nvfp4_f32out", False, False, 1),
    ("vib3_launch_partial_matmul_nvfp4_fp16in", True, True, 1),
    ("vib3_launch_fused_swiglu_nvfp4", False, True, 2),
    ("vib3_launch_fused_swiglu_nvfp4_f32out", False, False, 2),
])
def test_scalar_nvfp4_within_tolerance(entry, in16, out16, ns):
    from vib3_amd import _lib
    _say(f"case: {entry}")
    rng = np.random.default_rng(41 + ns)
    m, k = 520, 7168 if not in16 else 2048
    x = rng.standard_normal(k).astype(np.float32)
    if in16:
        x = x.astype(np.float16).astype(np.float32)
    mats = [rand_codes_scales(rng, m, k, e8m0=False) for _ in range(ns)]
    pages = [dev(np.concatenate([d, s.view(np.uint8).ravel()])) for d, s in mats]
    xd = torch.from_numpy(x.astype(np.float16) if in16 else x).cuda()
    out = torch.zeros(m, dtype=torch.float16 if out16 else torch.float32, device="cuda")
    ptrs = []
    for (d, _), p in zip(mats, pages):
        ptrs += [p.data_ptr(), p.data_ptr() + d.size]
    _lib.call(entry, xd.data_ptr(), *ptrs, out.data_ptr(), k, m, 32, _st())
    torch.cuda.synchronize()
    sums = [O.nvfp4_seq_matvec_f64(x, d, s, m, k) for d, s in mats]
    want = sums[0] if ns == 1 else sums[1] / (1 + np.exp(-sums[1])) * sums[0]
    got = out.cpu().numpy().astype(np.float64)
    if out16:
        w16 = want.astype(np.float16).astype(np.float64)
        assert np.all(np.abs(got - w16) <= np.abs(w16) * 2.0 ** -10 + 2.0 ** -24 + 1e-6 * np.abs(want).max())
    else:
        assert rel_l2(got, want) <= 1e-6


def tiled_expert(rng, k_in, m_mid, m_out):
    mats = []
    for rows, k in ((m_mid, k_in), (m_mid, k_in), (m_out, m_mid)):
        d, s = rand_codes_scales(rng, rows, k, e8m0=False)
        mats.append((d, s, dev(np.concatenate([d, s.view(np.uint8).ravel()]))))
    return mats


def test_expert_batched_bit_exact():
    """kernels.cu:4708 at the Kimi shape: one expert, layer_output += w * down(...)."""
    from vib3_amd import kernels as K
    _say("case: expert_batched kimi")
    rng = np.random.default_rng(51)
    mats = tiled_expert(rng, 7168, 2048, 7168)
    x, codes, sc = quantized_act(rng, 7168)
    out0 = rng.standard_normal(7168).astype(np.float32)
    out = torch.from_numpy(out0.copy()).cuda()
    K.expert_batched(dev(codes), dev(sc), mats[0][2], mats[1][2], mats[2][2], out, 0.37,
                     7168, 2048, 7168)
    torch.cuda.synchronize()
    want = out0.copy()
    O.moe_experts_fused(codes, sc, [tuple((d, s) for d, s, _ in mats)], [0.37], 7168, 2048, 7168,
                        want)
    assert np.array_equal(out.cpu().numpy(), want)


def test_quantizer_chain_into_fused_path():
    """f16 weights -> vib3_launch_fp16_to_nvfp4_weight -> vib3_launch_repack_row_to_tiled ->
    the fused path, bit-exact with the oracle of every step; and the reference CPU quantizer's
    pages (kernels.rs:4085, FP16 scales) through the reference repacks into the same fused
    path, read as the reference's kernels read them (the scale's bits 7..14 as E8M0)."""
    from vib3_amd import _lib, kernels as K
    _say("case: quantizer chain -> fused")
    rng = np.random.default_rng(61)
    k_in, m_mid, m_out = 1024, 512, 1024
    dims = ((m_mid, k_in), (m_mid, k_in), (m_out, m_mid))
    x, codes, sc = quantized_act(rng, k_in)
    for mode in ("gpu_quantizer", "cpu_quantizer"):
        host, pages = [], []
        for rows, k in dims:
            w = (rng.standard_normal(rows * k) * 0.05).astype(np.float16)
            if mode == "gpu_quantizer":
                d = torch.zeros(rows * k // 2, dtype=torch.uint8, device="cuda")
                s = torch.zeros(rows * k // 32, dtype=torch.int16, device="cuda")
                wd = dev(w.view(np.uint16), np.uint16)
                _lib.call("vib3_launch_fp16_to_nvfp4_weight", wd.data_ptr(), d.data_ptr(),
                          s.data_ptr(), rows, k, _st())
                rd, rs = O.fp16_to_nvfp4_weight(w.view(np.uint16), rows, k)
            else:
                page = O.quantize_half_to_nvfp4(w.view(np.uint16), O.F16, rows, k)
                d = dev(page[: rows * k // 2])
                s = dev(page[rows * k // 2:])
                K.repack_weights_inplace(d, rows * k // 2)
                rd = O.fp4_split_half(page[: rows * k // 2])
                rs = page[rows * k // 2:].view(np.uint16)
            tmp = torch.empty(rows * k // 2, dtype=torch.uint8, device="cuda")
            K.repack_row_to_tiled(d, tmp, rows, k)
            torch.cuda.synchronize()
            assert np.array_equal(s.cpu().numpy().view(np.uint16).ravel(), rs)
            td = O.fp4_to_tiled(rd, rows, k)
            assert np.array_equal(d.cpu().numpy(), td)
            host.append((td, rs))
            pages.append((d, s))
        out = torch.zeros(m_out, dtype=torch.float32, device="cuda")
        a, asc = dev(codes), dev(sc)
        one = lambda v: (C.c_void_p * 1)(v)  # noqa: E731
        ptrs = [one(pages[i][j].data_ptr()) for i in range(3) for j in range(2)]
        _lib.call("vib3_launch_moe_experts_fused", a.data_ptr(), asc.data_ptr(), *ptrs,
                  (C.c_float * 1)(0.5), 1, k_in, m_mid, m_mid, m_out, out.data_ptr(), _st())
        torch.cuda.synchronize()
        want = np.zeros(m_out, dtype=np.float32)
        O.moe_experts_fused(codes, sc, [tuple(host)], [0.5], k_in, m_mid, m_out, want)
        assert np.array_equal(out.cpu().numpy(), want), mode


def test_fused_ws_two_streams_concurrently():
    """vib3_launch_moe_experts_fused_gpu_ws on two streams at once, each with its own
    workspace and inputs: each result equals the oracle's."""
    from vib3_amd import _lib
    _say("case: fused _ws two streams")
    rng = np.random.default_rng(71)
    E, k_in, m_mid, m_out = 16, 2048, 1024, 2048
    table = np.zeros((1, E, 3), dtype=np.uint64)
    keep, host = [], {}
    for e in range(E):
        mats = tiled_expert(rng, k_in, m_mid, m_out)
        host[e] = tuple((d, s) for d, s, _ in mats)
        for i, (_, _, p) in enumerate(mats):
            keep.append(p)
            table[0, e, i] = p.data_ptr()
    tab = torch.from_numpy(table.view(np.int64)).cuda()
    n_ws = _lib.load().vib3_moe_experts_fused_workspace_bytes(m_mid)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cases = []
    for si in range(2):
        ids = rng.choice(E, 4, replace=False).astype(np.uint16)
        wts = rng.uniform(0.1, 0.5, 4).astype(np.float32)
        x, codes, sc = quantized_act(rng, k_in)
        out0 = rng.standard_normal(m_out).astype(np.float32)
        cases.append(dict(ids=ids, wts=wts, codes=codes, sc=sc, out0=out0,
                          d_ids=dev(ids.view(np.uint8)), d_w=torch.from_numpy(wts).cuda(),
                          d_c=dev(codes), d_s=dev(sc), out=torch.from_numpy(out0.copy()).cuda(),
                          ws=torch.zeros(n_ws + 256, dtype=torch.uint8, device="cuda")))
    torch.cuda.synchronize()
    for rep in range(3):
        for si, c in enumerate(cases):
            c["out"].copy_(torch.from_numpy(c["out0"]))
        torch.cuda.synchronize()
        for si, c in enumerate(cases):
            ws = (c["ws"].data_ptr() + 255) // 256 * 256
            _lib.call("vib3_launch_moe_experts_fused_gpu_ws", c["d_c"].data_ptr(),
                      c["d_s"].data_ptr(), tab.data_ptr(), c["d_ids"].data_ptr(),
                      c["d_w"].data_ptr(), 0, E, 4, k_in, m_mid, m_mid, m_out,
                      c["out"].data_ptr(), ws, n_ws, streams[si].cuda_stream)
        torch.cuda.synchronize()
        for c in cases:
            want = c["out0"].copy()
            O.moe_experts_fused(c["codes"], c["sc"], [host[int(e)] for e in c["ids"]],
                                [float(w) for w in c["wts"]], k_in, m_mid, m_out, want)
            assert np.array_equal(c["out"].cpu().numpy(), want)


def test_fused_allocates_lazily_without_prewarm():
    """A process that never calls vib3_moe_prewarm_gpu_bufs: the first host-pointer launch
    allocates the intermediate buffer (the reference's ensure_moe_bufs) and computes the
    oracle's result; a launch under graph capture without it returns VIB3_ERR_WORKSPACE."""
    _say("case: fused lazy allocation (subprocess)")
    code = r'''
import sys; sys.path.insert(0, sys.argv[1])
import numpy as np, torch
from oracle import oracle as O
from vib3_amd import _lib, kernels as K
from tests.test_gpu_fp4_pages import tiled_expert, quantized_act, dev
rng = np.random.default_rng(81)
k_in, m_mid, m_out = 1024, 512, 1024
# graph capture first: nothing allocated yet on this device -> -4, nothing recorded
mats = tiled_expert(rng, k_in, m_mid, m_out)
x, codes, sc = quantized_act(rng, k_in)
a, asc = dev(codes), dev(sc)
out = torch.zeros(m_out, dtype=torch.float32, device="cuda")
torch.cuda.synchronize()
s = torch.cuda.Stream()
lib = _lib.load()
import ctypes as C
arr = lambda v: (C.c_void_p * 1)(v)
args = [a.data_ptr(), asc.data_ptr()]
for i in range(3):
    args += [arr(mats[i][2].data_ptr()), arr(mats[i][2].data_ptr() + mats[i][0].size)]
w = (C.c_float * 1)(0.75)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    rc = lib.vib3_launch_moe_experts_fused(*args, w, 1, k_in, m_mid, m_mid, m_out,
                                           out.data_ptr(), C.c_void_p(s.cuda_stream))
assert rc == -4, rc
rc = lib.vib3_launch_moe_experts_fused(*args, w, 1, k_in, m_mid, m_mid, m_out, out.data_ptr(),
                                       C.c_void_p(torch.cuda.current_stream().cuda_stream))
assert rc == 0, rc
torch.cuda.synchronize()
want = np.zeros(m_out, dtype=np.float32)
O.moe_experts_fused(codes, sc, [tuple((d, s) for d, s, _ in mats)], [0.75], k_in, m_mid, m_out, want)
assert np.array_equal(out.cpu().numpy(), want)
print("lazy ok")
'''
    r = subprocess.run([sys.executable, "-c", code, ROOT], capture_output=True, text=True,
                       timeout=180, cwd=ROOT)
    assert r.returncode == 0 and "lazy ok" in r.stdout, r.stdout + r.stderr
