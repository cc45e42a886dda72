"""The HIP kernels against the committed golden fixtures (tests/golden/fixtures.npz), through the
C ABI. Inputs are regenerated on the device by the library's generator (equal, bit for bit, to
the oracle's; tests/test_gpu_kernels.py checks that). Bars as in the other GPU tests: GEMV /
SwiGLU rel-L2 <= 5e-5, router ids exact and weights within 1e-6, layer rel-L2 <= 1e-3, MXFP4
batch rel-L2 <= 1e-3 per token with almost every bf16 output equal."""
import ctypes as C
import json
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
HERE = os.path.dirname(os.path.abspath(__file__))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def load():
    f = np.load(os.path.join(HERE, "golden", "fixtures.npz"))
    return f, json.loads(str(f["meta"]))


def lib():
    from vib3_amd import _lib
    return _lib


def st():
    return torch.cuda.current_stream().cuda_stream


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def dev_act(seed, stream, n):
    x = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    lib().call("vib3_synth_normal", x.data_ptr(), O.BF16, n, seed, stream, 0, 1.0, st())
    return x


def dev_int4_page(seed, stream, k, m, g, sdt, sigma):
    pk, ng = (k + 1) // 2, (k + g - 1) // g
    buf = torch.empty(m * pk + m * ng * 2, dtype=torch.uint8, device="cuda")
    lib().call("vib3_synth_int4_page", buf.data_ptr(), seed, stream, k, g, sdt, float(sigma), 0, m,
               st())
    return buf


def test_gemv_and_swiglu_fixtures():
    _say("[golden] gemv / swiglu")
    f, meta = load()
    for name in ("gemv_bf16_g32", "gemv_f16_g128"):
        m = meta[name]
        seed, stream, sigma = m["page"]
        page = dev_int4_page(seed, stream, m["k"], m["m"], m["g"], m["scale_dt"], sigma)
        x = dev_act(m["x"][0], m["x"][1], m["k"])
        out = torch.empty(m["m"], dtype=torch.float32, device="cuda")
        lib().call("vib3_launch_partial_matmul_int4_ex", x.data_ptr(), O.BF16, page.data_ptr(),
                   out.data_ptr(), O.F32, m["k"], m["m"], m["g"], m["scale_dt"], st())
        torch.cuda.synchronize()
        assert rel_l2(out.cpu().numpy(), f[name]) <= 5e-5, name
    m = meta["swiglu_bf16_g32"]
    up = dev_int4_page(m["up"][0], m["up"][1], m["k"], m["m"], m["g"], m["scale_dt"], m["up"][2])
    gate = dev_int4_page(m["gate"][0], m["gate"][1], m["k"], m["m"], m["g"], m["scale_dt"],
                         m["gate"][2])
    x = dev_act(m["x"][0], m["x"][1], m["k"])
    out = torch.empty(m["m"], dtype=torch.float32, device="cuda")
    lib().call("vib3_launch_partial_swiglu_int4_ex", x.data_ptr(), O.BF16, up.data_ptr(),
               gate.data_ptr(), out.data_ptr(), O.F32, m["k"], m["m"], m["g"], m["scale_dt"], st())
    torch.cuda.synchronize()
    assert rel_l2(out.cpu().numpy(), f["swiglu_bf16_g32"]) <= 5e-5


def test_router_fixture():
    _say("[golden] router")
    f, meta = load()
    m = meta["router"]
    E, D, k = m["E"], m["D"], m["top_k"]
    w = torch.empty(E * D, dtype=torch.float32, device="cuda")
    lib().call("vib3_synth_normal", w.data_ptr(), O.F32, E * D, m["w"][0], m["w"][1], 0, m["w"][2],
               st())
    b = torch.empty(E, dtype=torch.float32, device="cuda")
    lib().call("vib3_synth_normal", b.data_ptr(), O.F32, E, m["bias"][0], m["bias"][1], 0,
               m["bias"][2], st())
    x = dev_act(m["x"][0], m["x"][1], D)
    ws = torch.zeros(lib().load().vib3_router_workspace_bytes(E), dtype=torch.uint8, device="cuda")
    ids = torch.empty(k, dtype=torch.int16, device="cuda")
    wts = torch.empty(k, dtype=torch.float32, device="cuda")
    sc = torch.empty(E, dtype=torch.float32, device="cuda")
    lib().call("vib3_launch_router_topk_ex", x.data_ptr(), O.BF16, w.data_ptr(), O.F32, b.data_ptr(),
               D, E, k, m["mode"], m["scaling"], m["normalize"], sc.data_ptr(), ids.data_ptr(),
               wts.data_ptr(), ws.data_ptr(), st())
    torch.cuda.synchronize()
    assert ids.cpu().numpy().astype(np.int64).tolist() == list(f["router_ids"])
    assert np.allclose(wts.cpu().numpy(), f["router_wts"], rtol=1e-6, atol=1e-7)
    assert rel_l2(sc.cpu().numpy(), f["router_scores"]) <= 1e-6


def test_layer_fixture():
    _say("[golden] small MoE layer (given ids)")
    from vib3_amd._lib import MoeInt4Layer
    f, meta = load()
    m = meta["layer"]
    seed, hidden, inter, g, sdt = m["x"][0], m["hidden"], m["inter"], m["g"], m["scale_dt"]
    n_routed = m["experts"] - len(m["shared"])
    pages = {e: [dev_int4_page(seed, 100 + 3 * e + s, *((hidden, inter) if s < 2 else (inter, hidden)),
                               g, sdt, m["sigma"]) for s in range(3)] for e in range(m["experts"])}
    table = torch.tensor([[pages[e][s].data_ptr() for s in range(3)] for e in range(n_routed)],
                         dtype=torch.int64, device="cuda")
    shared = torch.tensor([[pages[e][s].data_ptr() for s in range(3)] for e in m["shared"]],
                          dtype=torch.int64, device="cuda")
    x = dev_act(seed, m["x"][1], hidden)
    ids = torch.from_numpy(f["layer_ids"].astype(np.int16)).cuda()
    wts = torch.from_numpy(f["layer_wts"]).cuda()
    out = torch.empty(hidden, dtype=torch.float32, device="cuda")
    L = MoeInt4Layer()
    L.x, L.x_dtype, L.hidden, L.inter, L.group_size, L.scale_dtype = x.data_ptr(), O.BF16, hidden, inter, g, sdt
    L.num_experts, L.top_k = n_routed, ids.numel()
    L.in_ids, L.in_weights = ids.data_ptr(), wts.data_ptr()
    L.page_table, L.shared_page_table, L.num_shared = table.data_ptr(), shared.data_ptr(), len(m["shared"])
    L.max_pages = 1
    L.rows_per_page[0], L.rows_per_page[1], L.rows_per_page[2] = inter, inter, hidden
    L.out = out.data_ptr()
    n = lib().load().vib3_moe_int4_workspace_bytes(C.byref(L))
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda")
    L.workspace, L.workspace_bytes = ws.data_ptr(), n
    lib().call("vib3_launch_moe_int4_layer", C.byref(L), st())
    torch.cuda.synchronize()
    assert rel_l2(out.cpu().numpy(), f["layer_out"]) <= 1e-3


def test_mxfp4_fixture():
    _say("[golden] batched MXFP4 MoE")
    from vib3_amd._lib import MoeMxfp4Batch
    f, meta = load()
    m = meta["mxfp4"]
    seed, hidden, inter, E, T, k = m["x"][0], m["hidden"], m["inter"], m["E"], m["tokens"], m["top_k"]
    pages = []
    for e in range(E):
        row = []
        for s in range(3):
            rows, kk = (inter, hidden) if s < 2 else (hidden, inter)
            buf = torch.empty(rows * kk // 2 + rows * kk // 32, dtype=torch.uint8, device="cuda")
            lib().call("vib3_synth_mxfp4_page", buf.data_ptr(), seed, 200 + 3 * e + s, kk, 0, rows,
                       st())
            row.append(buf)
        pages.append(row)
    table = torch.tensor([[p.data_ptr() for p in row] for row in pages], dtype=torch.int64,
                         device="cuda")
    x = dev_act(seed, m["x"][1], T * hidden)
    ids = torch.from_numpy(f["mxfp4_ids"].astype(np.int16)).cuda()
    wts = torch.from_numpy(f["mxfp4_wts"]).cuda()
    out = torch.empty((T, hidden), dtype=torch.bfloat16, device="cuda")
    d = MoeMxfp4Batch()
    d.x, d.tokens, d.hidden, d.inter, d.num_experts, d.top_k = x.data_ptr(), T, hidden, inter, E, k
    d.ids, d.weights, d.page_table, d.out = ids.data_ptr(), wts.data_ptr(), table.data_ptr(), out.data_ptr()
    n = lib().load().vib3_moe_mxfp4_workspace_bytes(C.byref(d))
    ws = torch.zeros(n + 256, dtype=torch.uint8, device="cuda")
    d.workspace = (ws.data_ptr() + 255) // 256 * 256
    d.workspace_bytes = n
    lib().call("vib3_launch_moe_mxfp4_batched", C.byref(d), st())
    torch.cuda.synchronize()
    got_bits = out.view(torch.int16).cpu().numpy().view(np.uint16)
    ref_bits = f["mxfp4_out_bf16"]
    got = O.to_f32(got_bits.ravel(), O.BF16).reshape(T, hidden)
    ref = O.to_f32(ref_bits.ravel(), O.BF16).reshape(T, hidden)
    for t in range(T):
        assert rel_l2(got[t], ref[t]) <= 1e-3, t
    assert np.mean(got_bits == ref_bits) > 0.97


def test_rmsnorm_fixture():
    """vib3_launch_rms_norm_f32 against the fixture: within 2 ulp (the same summation order;
    sqrt and divide correctly rounded on both sides)."""
    _say("[golden] RMSNorm")
    from vib3_amd import kernels as K
    f, meta = load()
    m = meta["rmsnorm"]
    seed, stream, sigma = m["x"]
    x = O.synth_normal_array(seed, stream, 0, m["n"], sigma, O.F32)
    wseed, wstream, wsigma, woff = m["w"]
    w = (O.synth_normal_array(wseed, wstream, 0, m["n"], wsigma, O.F32) + np.float32(woff)).astype(
        np.float16)
    out = torch.empty(m["n"], dtype=torch.float32, device="cuda")
    K.rms_norm_f32(torch.from_numpy(x).cuda(), out, torch.from_numpy(w).cuda(), m["n"], m["eps"])
    torch.cuda.synchronize()
    ref = f["rmsnorm_out"]
    assert np.all(np.abs(out.cpu().numpy() - ref) <= 2 * np.spacing(np.abs(ref)))
