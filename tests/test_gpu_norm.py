"""GPU parity of the operations either side of the MoE sublayer (engine.rs:5064-5307): the
pre-MoE RMSNorm, the residual add, the shared expert's sigmoid gate, standalone (the reference
C ABI) and inside the fused layer.

Bars: RMSNorm within 2 f32 ulp of the oracle (same summation order; sqrt and divide are
correctly rounded on both sides); f16 output within one f16 ulp; residual add bit-exact; the
gated accumulate within 1e-6 relative (device expf against libm); layer outputs rel-L2 <= 1e-3
against the oracle's composition RMSNorm -> router -> experts (shared experts weighted by
sigmoid(xn . gate)) -> + residual, router ids bit-exact where the margin exceeds 1e-3.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 0x5EED0006


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _f32(n, stream, sigma):
    return O.synth_normal_array(SEED, stream, 0, n, sigma, O.F32)


def _f16(n, stream, sigma, offset=0.0):
    v = O.synth_normal_array(SEED, stream, 0, n, sigma, O.F32) + np.float32(offset)
    return v.astype(np.float16).view(np.uint16)


def _dev16(bits):
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.float16)


@pytest.mark.parametrize("n,sigma,eps", [(7168, 30.0, 1e-6), (4096, 1.0, 1e-5), (1000, 1e-4, 1e-6),
                                         (1, 2.0, 1e-6)])
def test_rms_norm_f32_matches_oracle(n, sigma, eps):
    """Residual-stream magnitudes (L2 ~ 2500), unit scale, eps-dominated tiny values, n = 1."""
    from vib3_amd import kernels as K
    _say(f"case: rms_norm n={n} sigma={sigma} eps={eps}")
    x = _f32(n, 1, sigma)
    w = _f16(n, 2, 0.1, 1.0)
    xd, wd = torch.from_numpy(x).cuda(), _dev16(w)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    K.rms_norm_f32(xd, out, wd, n, eps)
    out16 = torch.empty(n, dtype=torch.float16, device="cuda")
    K.rms_norm_f32_to_f16(xd, out16, wd, n, eps)
    torch.cuda.synchronize()
    ref = O.rms_norm_f32(x, w, eps)
    got = out.cpu().numpy()
    ulp = np.spacing(np.abs(ref).astype(np.float32))
    assert np.all(np.abs(got - ref) <= 2 * ulp), float(np.max(np.abs(got - ref) / ulp))
    ref16 = ref.astype(np.float16)
    got16 = out16.cpu().numpy()
    assert np.all(np.abs(got16.astype(np.float32) - ref16.astype(np.float32))
                  <= np.spacing(np.abs(ref16)).astype(np.float32))


def test_residual_add_and_gated_accumulate():
    from vib3_amd import kernels as K
    n = 7168
    acc = _f32(n, 3, 40.0)
    lo = _f32(n, 4, 1.0)
    a = torch.from_numpy(acc.copy()).cuda()
    K.residual_add_f32_f32(a, torch.from_numpy(lo).cuda(), n)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), O.residual_add_f32(acc, lo))

    e = _f16(n, 5, 0.5)
    for g in (-3.0, 0.0, 0.7):
        o = torch.from_numpy(acc.copy()).cuda()
        K.sigmoid_gated_accumulate_f32(o, _dev16(e),
                                       torch.tensor([g], dtype=torch.float32, device="cuda"), n)
        torch.cuda.synchronize()
        sg = np.float32(O.sigmoid(g))
        ref = acc + sg * e.view(np.float16).astype(np.float32)  # f32 product, then f32 add
        assert np.allclose(o.cpu().numpy(), ref, rtol=1e-6, atol=1e-6)


def _shape(moe, DT_BF16, hidden, inter, E, ns):
    return moe.BankShape(hidden=hidden, inter=inter, group_size=32, scale_dtype=DT_BF16,
                         scale_sigma=0.03, num_experts=E, num_shared=ns)


@pytest.mark.parametrize("hidden,inter,E,k,ns,layout,use_norm,use_gate,use_res", [
    (1024, 256, 16, 4, 2, "contiguous", True, True, True),
    (1024, 256, 16, 4, 2, "paged", True, True, False),
    (2048, 512, 40, 6, 1, "contiguous", False, True, True),
    (2048, 512, 40, 6, 1, "contiguous", True, False, True),
    (7168, 2048, 384, 8, 1, "contiguous", True, True, True),  # Kimi-K2.5 shape
])
def test_layer_with_norm_gate_residual(hidden, inter, E, k, ns, layout, use_norm, use_gate,
                                       use_res):
    from vib3_amd import moe
    from vib3_amd._lib import DT_BF16, ROUTER_SIGMOID
    _say(f"case: layer hidden={hidden} E={E} k={k} shared={ns} {layout} norm={use_norm} "
         f"gate={use_gate} residual={use_res}")
    sh = _shape(moe, DT_BF16, hidden, inter, E, ns)
    bank = moe.Int4ExpertBank(sh, layer=1, seed=SEED, layout=layout, tile_rows=64,
                              pool_bytes=256 << 20 if layout == "paged" else None)
    w, bias = moe.make_router(sh, 1, SEED, 0.02, 0.1)
    eps = 1e-6
    nw = _f16(hidden, 10, 0.1, 1.0)
    gw = _f16(ns * hidden, 11, 0.02)
    layer = moe.MoeInt4Layer(bank, w, bias, top_k=k, scoring_mode=ROUTER_SIGMOID,
                             scaling_factor=2.827, normalize=True,
                             norm_weight=_dev16(nw) if use_norm else None, norm_eps=eps,
                             shared_gate=_dev16(gw) if use_gate else None)
    # the f32 residual stream (large, as between decoder layers) or a bf16 activation
    if use_norm:
        xh = _f32(hidden, 12, 20.0)
        x = torch.from_numpy(xh).cuda()
    else:
        x = moe.make_activation(hidden, 3, SEED)
        xh = x.float().cpu().numpy()
    res = _f32(hidden, 13, 20.0)
    out = layer.launch(x, residual=torch.from_numpy(res).cuda() if use_res else None)
    got = out.cpu().numpy()
    torch.cuda.synchronize()

    xn = O.rms_norm_f32(xh, nw, eps) if use_norm else xh
    r_ids, r_wts, r_scores = O.router(xn, w.cpu().numpy(), O.F32, E, hidden, k, 1, 2.827, True,
                                      bias.cpu().numpy())
    keys = np.sort(1 / (1 + np.exp(-r_scores.astype(np.float64))) + bias.cpu().numpy())[::-1]
    assert keys[k - 1] - keys[k] > 1e-3, "selection margin below 1e-3: choose another token"
    assert layer.ids.cpu().numpy().view(np.uint16)[:k].tolist() == r_ids.tolist()
    gates = None
    if use_gate:
        gates = np.array([O.sigmoid(O.linear_row_f16(xn, gw[s * hidden:(s + 1) * hidden]))
                          for s in range(ns)], dtype=np.float32)
    routed = {int(e): bank.expert_pages_host(int(e)) for e in r_ids}
    shared = [bank.expert_pages_host(E + s) for s in range(ns)]
    ref = O.moe_layer(xn, hidden, inter, 32, DT_BF16, routed, r_ids, r_wts, shared,
                      faithful=True, shared_weights=gates)
    if use_res:
        moe_part = rel_l2(got - res, ref)
        ref = O.residual_add_f32(res, ref)
        _say(f"  sublayer rel_l2={moe_part:.3e}")
        assert moe_part <= 1e-3
    rel = rel_l2(got, ref)
    _say(f"  rel_l2={rel:.3e}")
    assert rel <= 1e-3


def test_in_place_residual_stream():
    """The engine's in-place form (engine.rs:5302): x, residual and out all the same f32
    hidden_state buffer. The result equals the out-of-place launch bit for bit."""
    from vib3_amd import moe
    from vib3_amd._lib import DT_BF16, ROUTER_SIGMOID
    _say("case: in-place residual stream")
    sh = _shape(moe, DT_BF16, 1024, 256, 16, 1)
    bank = moe.Int4ExpertBank(sh, layer=4, seed=SEED)
    w, bias = moe.make_router(sh, 4, SEED, 0.02, 0.1)
    layer = moe.MoeInt4Layer(bank, w, bias, top_k=4, scoring_mode=ROUTER_SIGMOID,
                             scaling_factor=2.827, norm_weight=_dev16(_f16(1024, 10, 0.1, 1.0)),
                             shared_gate=_dev16(_f16(1024, 11, 0.02)))
    xh = _f32(1024, 14, 20.0)
    ref = layer.launch(torch.from_numpy(xh).cuda(),
                       residual=torch.from_numpy(xh).cuda()).cpu().numpy().copy()
    hs = torch.from_numpy(xh.copy()).cuda()
    d = layer._desc(hs)
    d.residual = hs.data_ptr()
    d.out = hs.data_ptr()
    from vib3_amd import _lib
    assert _lib.load().vib3_launch_moe_int4_layer(
        d, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert np.array_equal(hs.cpu().numpy(), ref)


def test_norm_needs_f32_stream():
    from vib3_amd import moe
    from vib3_amd._lib import DT_BF16, ROUTER_SIGMOID, Vib3Error
    sh = _shape(moe, DT_BF16, 1024, 256, 8, 1)
    bank = moe.Int4ExpertBank(sh, layer=2, seed=SEED)
    w, bias = moe.make_router(sh, 2, SEED, 0.02, 0.1)
    layer = moe.MoeInt4Layer(bank, w, bias, top_k=2, scoring_mode=ROUTER_SIGMOID,
                             norm_weight=_dev16(_f16(1024, 10, 0.1, 1.0)))
    with pytest.raises(Vib3Error):
        layer.launch(moe.make_activation(1024, 0, SEED))  # bf16 x with a norm: unsupported


@pytest.mark.parametrize("hidden,inter,E,k,ns", [(1024, 256, 16, 4, 2), (7168, 2048, 384, 8, 1)])
def test_fused_prologue_equals_prologue_kernel(hidden, inter, E, k, ns):
    """The gate/up kernel that normalises x and computes the shared gates itself gives the
    layer of the separate prologue kernel bit for bit (same summation orders), over several
    tokens, with and without the residual."""
    from vib3_amd import moe
    from vib3_amd._lib import DT_BF16, MOE_SEPARATE_PROLOGUE, ROUTER_SIGMOID
    _say(f"case: fused prologue hidden={hidden} E={E} k={k} shared={ns}")
    sh = _shape(moe, DT_BF16, hidden, inter, E, ns)
    bank = moe.Int4ExpertBank(sh, layer=5, seed=SEED)
    w, bias = moe.make_router(sh, 5, SEED, 0.02, 0.1)
    layer = moe.MoeInt4Layer(bank, w, bias, top_k=k, scoring_mode=ROUTER_SIGMOID,
                             scaling_factor=2.827, normalize=True,
                             norm_weight=_dev16(_f16(hidden, 10, 0.1, 1.0)), norm_eps=1e-6,
                             shared_gate=_dev16(_f16(ns * hidden, 11, 0.02)))
    for t in range(3):
        x = torch.from_numpy(_f32(hidden, 20 + t, 20.0)).cuda()
        res = torch.from_numpy(_f32(hidden, 30 + t, 20.0)).cuda() if t != 1 else None
        flags = layer.flags
        fused = layer.launch(x, residual=res).cpu().numpy().copy()
        ids_f = layer.ids.cpu().numpy().copy()
        layer.flags = flags | MOE_SEPARATE_PROLOGUE
        sep = layer.launch(x, residual=res).cpu().numpy().copy()
        ids_s = layer.ids.cpu().numpy().copy()
        layer.flags = flags
        assert np.array_equal(ids_f, ids_s)
        assert np.array_equal(fused.view(np.uint32), sep.view(np.uint32)), t


def test_sublayer_graph_replay():
    """The whole sublayer (fused RMSNorm and shared gates in the gate/up kernel, residual in the
    down epilogue) captured once in a HIP graph and replayed for three tokens, with new x and
    residual copied in between: every replay equals an eager launch of the same token bit for
    bit, and the router status stays clean."""
    from vib3_amd import moe
    from vib3_amd._lib import DT_BF16, ROUTER_SIGMOID
    _say("case: sublayer graph capture + replays")
    hidden, ns = 1024, 2
    sh = _shape(moe, DT_BF16, hidden, 256, 16, ns)
    bank = moe.Int4ExpertBank(sh, layer=6, seed=SEED)
    w, bias = moe.make_router(sh, 6, SEED, 0.02, 0.1)
    kw = dict(top_k=4, scoring_mode=ROUTER_SIGMOID, scaling_factor=2.827, normalize=True,
              norm_weight=_dev16(_f16(hidden, 10, 0.1, 1.0)), norm_eps=1e-6,
              shared_gate=_dev16(_f16(ns * hidden, 11, 0.02)))
    layer = moe.MoeInt4Layer(bank, w, bias, **kw)
    eager = moe.MoeInt4Layer(bank, w, bias, **kw)
    xbuf = torch.from_numpy(_f32(hidden, 40, 20.0)).cuda()
    rbuf = torch.from_numpy(_f32(hidden, 41, 20.0)).cuda()
    side = torch.cuda.Stream()
    layer.launch(xbuf, residual=rbuf)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        layer.launch(xbuf, residual=rbuf, stream=side)
    torch.cuda.synchronize()
    seen = set()
    for t in range(3):
        xt = torch.from_numpy(_f32(hidden, 50 + t, 20.0)).cuda()
        rt = torch.from_numpy(_f32(hidden, 60 + t, 20.0)).cuda()
        xbuf.copy_(xt)
        rbuf.copy_(rt)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = layer.out.cpu().numpy().copy()
        ids = tuple(layer.ids.cpu().numpy().tolist())
        ref = eager.launch(xt, residual=rt).cpu().numpy().copy()
        _say(f"  replay {t}")
        assert ids == tuple(eager.ids.cpu().numpy().tolist())
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        seen.add(ids)
    assert len(seen) > 1
    assert layer.status() == 0
    del graph
