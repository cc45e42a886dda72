"""GPU parity of the reference's fused NVFP4 MoE entry points (vib3_launch_moe_experts_fused
and _gpu, kernels.cu:5650 / :5868), the FP4 activation quantizer and the page repacks, through
the C ABI (the Rust-API mirror in vib3_amd/kernels.py) against the CPU oracle.

Bar: bit-exact. Every group dot product is exact and the row sums are exact f64 rounded once,
and SwiGLU's exp is the same operation sequence on both sides, so GPU and oracle agree to the
bit. Weight pages are random tiled split-half bytes with bf16 scales of exponent 2^-8..2^-4
and random mantissa bits (which the reference's E8M0 decode drops)."""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _st():
    return torch.cuda.current_stream().cuda_stream


def random_page(rng, m, k):
    """Host page: tiled split-half data [m*k/2] then bf16 scales [m][k/32]."""
    data = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
    ew = rng.integers(119, 124, (m, k // 32))
    sc = ((ew << 7) | rng.integers(0, 128, (m, k // 32))).astype(np.uint16)
    return data, sc


def page_bytes(data, sc):
    return np.concatenate([data, sc.reshape(-1).view(np.uint8)])


def dev_u8(a):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()
    return t


def quantize_dev(x_host):
    from vib3_amd import kernels as K
    x = torch.from_numpy(x_host.astype(np.float32)).cuda()
    k = x_host.size
    codes = torch.zeros((k + 31) // 32 * 16, dtype=torch.uint8, device="cuda")
    sc = torch.zeros((k + 31) // 32, dtype=torch.uint8, device="cuda")
    K.quantize_activation_fp4(x, codes, sc, k)
    return x, codes, sc


@pytest.mark.parametrize("k", [7168, 4096, 2048 + 96])
def test_quantize_activation_bit_exact(k):
    _say(f"case: fp4 activation quantizer k={k}")
    rng = np.random.default_rng(k)
    x = rng.normal(0, 3, k).astype(np.float32)
    x[32:64] = 0.0
    x[96:128] *= np.float32(1e-20)
    x[160:192] *= np.float32(1e20)
    _, codes, sc = quantize_dev(x)
    rc, rs = O.fp4_quantize_act(x)
    assert np.array_equal(codes.cpu().numpy()[: rc.size], rc)
    assert np.array_equal(sc.cpu().numpy(), rs)


def test_repacks_bit_exact():
    from vib3_amd import kernels as K
    _say("case: fp4 repacks")
    rng = np.random.default_rng(1)
    m, k = 48, 512
    seq = rng.integers(0, 256, m * k // 2 + 8, dtype=np.uint8)  # a partial block at the end
    d = dev_u8(seq)
    K.repack_weights_inplace(d, seq.size)
    split = O.fp4_split_half(seq)
    assert np.array_equal(d.cpu().numpy(), split)
    row = dev_u8(split[: m * k // 2])
    tmp = torch.empty(m * k // 2, dtype=torch.uint8, device="cuda")
    K.repack_row_to_tiled(row, tmp, m, k)
    assert np.array_equal(row.cpu().numpy(), O.fp4_to_tiled(split[: m * k // 2], m, k))


class Fp4Layer:
    """Device pages of `n` selected experts of one layer plus the engine's page table
    u64[layers][E][3] (entries of unselected experts 0), and their host copies."""

    def __init__(self, rng, layers, E, layer, ids, k_in, m_mid, m_out):
        self.k_in, self.m_mid, self.m_out = k_in, m_mid, m_out
        self.host, self.dev = {}, []
        table = np.zeros((layers, E, 3), dtype=np.uint64)
        for e in sorted(set(int(i) for i in ids if i < E)):
            mats = (random_page(rng, m_mid, k_in), random_page(rng, m_mid, k_in),
                    random_page(rng, m_out, m_mid))
            self.host[e] = mats
            for s, (d, sc) in enumerate(mats):
                t = dev_u8(page_bytes(d, sc))
                self.dev.append(t)
                table[layer, e, s] = t.data_ptr()
        self.table_host = table
        self.table = torch.from_numpy(table.view(np.int64)).cuda()

    def oracle(self, codes, sc, ids, wts, out):
        experts = [self.host[int(e)] for e in ids if int(e) in self.host]
        w = [float(wt) for e, wt in zip(ids, wts) if int(e) in self.host]
        return O.moe_experts_fused(codes, sc, experts, w, self.k_in, self.m_mid, self.m_out, out)


def kimi_case(seed=7, ids=None):
    rng = np.random.default_rng(seed)
    E, layers, layer = 384, 2, 1
    if ids is None:
        ids = rng.choice(E, 8, replace=False).astype(np.uint16)
    lay = Fp4Layer(rng, layers, E, layer, ids, 7168, 2048, 7168)
    wts = rng.uniform(0.05, 0.5, len(ids)).astype(np.float32)
    x = rng.normal(0, 1, 7168).astype(np.float32)
    out0 = rng.normal(0, 1, 7168).astype(np.float32)
    return lay, ids, wts, x, out0, E, layer


def test_fused_gpu_kimi_shape_bit_exact():
    """Kimi-K2.5 shape (hidden 7168, expert inter 2048), 8 of 384 experts, layer 1 of a
    two-layer table, through vib3_launch_moe_experts_fused_gpu; layer_output accumulates."""
    from vib3_amd import kernels as K
    _say("case: fused_gpu kimi shape")
    lay, ids, wts, x, out0, E, layer = kimi_case()
    K.moe_prewarm_gpu_bufs(2048, 2048)
    _, codes, sc = quantize_dev(x)
    out = torch.from_numpy(out0.copy()).cuda()
    K.moe_experts_fused_gpu(codes, sc, lay.table, torch.from_numpy(ids.view(np.int16)).cuda(),
                            torch.from_numpy(wts).cuda(), layer, E, len(ids), 7168, 2048, 7168,
                            out)
    got = out.cpu().numpy()
    ref = lay.oracle(codes.cpu().numpy(), sc.cpu().numpy(), ids, wts, out0.copy())
    _say(f"  identical {np.mean(got == ref):.6f}, max |diff| {np.abs(got - ref).max():.3e}")
    assert np.array_equal(got, ref)

    # the host-pointer entry point on the same pages gives the same bits
    pages = []
    for e, w in zip(ids, wts):
        t = lay.table_host[layer, int(e)]
        pages.append((int(t[0]), int(t[1]), int(t[2]), float(w)))
    out2 = torch.from_numpy(out0.copy()).cuda()
    K.moe_experts_fused(codes, sc, pages, 7168, 2048, 7168, out2)
    assert np.array_equal(out2.cpu().numpy(), got)


@pytest.mark.parametrize("m_mid,odd_ids", [(256, False), (512, True)])
def test_fused_gpu_skips_unusable_slots_and_checks_arguments(m_mid, odd_ids):
    """An id >= num_experts_total and an id whose table entry is 0 contribute nothing;
    argument errors return the reference's codes (-2 more than 8 experts) or ours. M_mid 512
    takes the one-workgroup-per-CU down kernel (page addresses from the gate/up kernel's
    records); odd_ids passes the ids at an address that is 2 mod 4."""
    from vib3_amd import _lib
    from vib3_amd import kernels as K
    _say(f"case: fused_gpu unusable slots, errors, m_mid {m_mid}, odd ids {odd_ids}")
    rng = np.random.default_rng(11)
    k_in, m_out, E = 512, 256, 16
    ids = np.array([3, 40, 9, 5], dtype=np.uint16)  # 40 >= E; 5 gets no pages below
    lay = Fp4Layer(rng, 1, E, 0, ids[:3], k_in, m_mid, m_out)
    wts = np.array([0.5, 9.0, -0.25, 7.0], np.float32)
    x = rng.normal(0, 1, k_in).astype(np.float32)
    K.moe_prewarm_gpu_bufs(m_mid, m_mid)
    _, codes, sc = quantize_dev(x)
    out = torch.zeros(m_out, dtype=torch.float32, device="cuda")
    ids_dev = torch.from_numpy(np.concatenate([[7], ids]).astype(np.uint16).view(np.int16)).cuda()
    ids_dev = ids_dev[1:] if odd_ids else ids_dev[1:].clone()
    assert (ids_dev.data_ptr() % 4 == 2) == odd_ids
    K.moe_experts_fused_gpu(codes, sc, lay.table, ids_dev,
                            torch.from_numpy(wts).cuda(), 0, E, 4, k_in, m_mid, m_out, out)
    ref = lay.oracle(codes.cpu().numpy(), sc.cpu().numpy(), ids, wts,
                     np.zeros(m_out, np.float32))
    assert np.array_equal(out.cpu().numpy(), ref)
    # the host-pointer entry point: an expert whose pages are null contributes nothing either
    pages = [(int(lay.table_host[0, e][0]), int(lay.table_host[0, e][1]),
              int(lay.table_host[0, e][2]), float(w)) for e, w in zip(ids[[0, 2]], wts[[0, 2]])]
    pages.insert(1, (0, 0, 0, 9.0))
    out_h = torch.zeros(m_out, dtype=torch.float32, device="cuda")
    K.moe_experts_fused(codes, sc, pages, k_in, m_mid, m_out, out_h)
    ref_h = lay.oracle(codes.cpu().numpy(), sc.cpu().numpy(), ids[:3], wts[:3],
                       np.zeros(m_out, np.float32))
    assert np.array_equal(out_h.cpu().numpy(), ref_h)
    lib = _lib.load()
    args = lambda n, ki, mm, km, mo: (codes.data_ptr(), sc.data_ptr(), lay.table.data_ptr(),
                                      0, 0, 0, E, n, ki, mm, km, mo, out.data_ptr(), _st())
    assert lib.vib3_launch_moe_experts_fused_gpu(*args(9, k_in, m_mid, m_mid, m_out)) == -2
    assert lib.vib3_launch_moe_experts_fused_gpu(*args(2, k_in, m_mid, 128, m_out)) == -2
    assert lib.vib3_launch_moe_experts_fused_gpu(*args(2, 576, m_mid, m_mid, m_out)) == -1
    assert lib.vib3_launch_moe_experts_fused_gpu(*args(2, k_in, m_mid, m_mid, m_out)) == -3


def test_fused_from_converter_order_pages():
    """Pages in the converter's sequential nibble order, repacked on the device by the
    reference-named repacks (split-half in place, then row -> tiled) as engine.rs:1165-1230
    does, then the fused layer: equal to the oracle over the oracle's repack."""
    from vib3_amd import kernels as K
    _say("case: fused from sequential pages")
    rng = np.random.default_rng(12)
    k_in, m_mid, m_out, E = 1024, 512, 1024, 6
    ids = np.array([4, 1, 2], dtype=np.uint16)
    table = np.zeros((1, E, 3), dtype=np.uint64)
    keep, host = [], {}
    for e in ids:
        mats = []
        for s, (m, k) in enumerate([(m_mid, k_in), (m_mid, k_in), (m_out, m_mid)]):
            seq = rng.integers(0, 256, m * k // 2, dtype=np.uint8)
            _, sc = random_page(rng, m, k)
            page = dev_u8(page_bytes(seq, sc))
            tmp = torch.empty(m * k // 2, dtype=torch.uint8, device="cuda")
            K.repack_weights_inplace(page, m * k // 2)
            K.repack_row_to_tiled(page, tmp, m, k)
            keep.append(page)
            table[0, e, s] = page.data_ptr()
            mats.append((O.fp4_to_tiled(O.fp4_split_half(seq), m, k), sc))
        host[int(e)] = mats
    wts = np.array([0.3, 0.2, 0.5], np.float32)
    x = rng.normal(0, 1, k_in).astype(np.float32)
    K.moe_prewarm_gpu_bufs(m_mid, m_mid)
    _, codes, sc = quantize_dev(x)
    out = torch.zeros(m_out, dtype=torch.float32, device="cuda")
    K.moe_experts_fused_gpu(codes, sc, torch.from_numpy(table.view(np.int64)).cuda(),
                            torch.from_numpy(ids.view(np.int16)).cuda(),
                            torch.from_numpy(wts).cuda(), 0, E, 3, k_in, m_mid, m_out, out)
    ref = O.moe_experts_fused(codes.cpu().numpy(), sc.cpu().numpy(), [host[int(e)] for e in ids],
                              wts, k_in, m_mid, m_out, np.zeros(m_out, np.float32))
    assert np.array_equal(out.cpu().numpy(), ref)


def test_fused_gpu_graph_replay():
    """quantize + fused_gpu captured once (the engine's decode graph, engine.rs:5018-5033) and
    replayed for new activations, ids and weights: each replay equals the eager result."""
    from vib3_amd import kernels as K
    _say("case: fused_gpu graph replay")
    rng = np.random.default_rng(13)
    k_in, m_mid, m_out, E = 2048, 512, 2048, 24
    all_ids = np.arange(E, dtype=np.uint16)
    lay = Fp4Layer(rng, 1, E, 0, all_ids, k_in, m_mid, m_out)
    K.moe_prewarm_gpu_bufs(m_mid, m_mid)
    x = torch.zeros(k_in, dtype=torch.float32, device="cuda")
    codes = torch.zeros(k_in // 2, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(k_in // 32, dtype=torch.uint8, device="cuda")
    ids = torch.zeros(4, dtype=torch.int16, device="cuda")
    wts = torch.zeros(4, dtype=torch.float32, device="cuda")
    out = torch.zeros(m_out, dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()

    def step():
        K.quantize_activation_fp4(x, codes, sc, k_in)
        K.moe_experts_fused_gpu(codes, sc, lay.table, ids, wts, 0, E, 4, k_in, m_mid, m_out, out)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step()
    for t in range(3):
        xi = rng.normal(0, 1, k_in).astype(np.float32)
        ii = rng.choice(E, 4, replace=False).astype(np.uint16)
        wi = rng.uniform(0, 1, 4).astype(np.float32)
        x.copy_(torch.from_numpy(xi))
        ids.copy_(torch.from_numpy(ii.view(np.int16)))
        wts.copy_(torch.from_numpy(wi))
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().copy()
        out.zero_()
        step()
        torch.cuda.synchronize()
        assert np.array_equal(got, out.cpu().numpy())
        rc, rs = O.fp4_quantize_act(xi)
        ref = lay.oracle(rc, rs, ii, wi, np.zeros(m_out, np.float32))
        assert np.array_equal(got, ref)
    del graph


@pytest.mark.parametrize("k,sigma,f16", [(7168, 20.0, True), (7168, 1.0, False), (3072, 5.0, True),
                                         (96, 0.5, True), (9216, 2.0, False)])
def test_fused_rms_norm_quantize_bit_exact(k, sigma, f16):
    """kernels.cu:6585 fused RMSNorm + FP4 quantize (vib3_launch_fused_rms_norm_quantize_fp4):
    codes, scales and the optional f16 output equal the oracle's bit for bit, for a residual-
    stream magnitude, unit and small inputs, one workgroup (k = 96) and k above the single-load
    form (9216)."""
    from vib3_amd import kernels as K
    _say(f"case: fused rms norm + fp4 quantize k={k} sigma={sigma} f16={f16}")
    rng = np.random.default_rng(k + int(sigma))
    x = rng.normal(0, sigma, k).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    xd = torch.from_numpy(x).cuda()
    wd = torch.from_numpy(w).cuda()
    codes = torch.zeros(k // 2, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(k // 32, dtype=torch.uint8, device="cuda")
    h = torch.zeros(k, dtype=torch.float16, device="cuda") if f16 else None
    K.fused_rms_norm_quantize_fp4(xd, wd, codes, sc, h, k, 1e-6)
    torch.cuda.synchronize()
    ref = O.fused_rms_norm_quantize_fp4(x, w.view(np.uint16), 1e-6, f16_out=f16)
    assert np.array_equal(codes.cpu().numpy(), ref[0])
    assert np.array_equal(sc.cpu().numpy(), ref[1])
    if f16:
        assert np.array_equal(h.cpu().numpy().view(np.uint16), ref[2])


def test_fused_rms_norm_quantize_errors():
    from vib3_amd import _lib
    lib = _lib.load()
    x = torch.zeros(64, dtype=torch.float32, device="cuda")
    w = torch.zeros(64, dtype=torch.float16, device="cuda")
    c = torch.zeros(32, dtype=torch.uint8, device="cuda")
    s = torch.zeros(2, dtype=torch.uint8, device="cuda")
    f = lib.vib3_launch_fused_rms_norm_quantize_fp4
    assert f(x.data_ptr(), w.data_ptr(), c.data_ptr(), s.data_ptr(), None, 0, 1e-6, _st()) != 0
    assert f(x.data_ptr(), w.data_ptr(), c.data_ptr(), s.data_ptr(), None, 48, 1e-6, _st()) != 0
    assert f(None, w.data_ptr(), c.data_ptr(), s.data_ptr(), None, 64, 1e-6, _st()) != 0
    assert f(x.data_ptr(), w.data_ptr(), c.data_ptr(), s.data_ptr(), None, 64, 1e-6, _st()) == 0
    torch.cuda.synchronize()
