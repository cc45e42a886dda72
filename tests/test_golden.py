"""The committed golden fixtures (tests/golden/fixtures.npz, written by
tests/golden/make_golden.py after an independent float64 check) reproduced bit for bit by the
oracle and its input generator: any change to either shows up here."""
import json
import os

import numpy as np

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


def load():
    f = np.load(os.path.join(HERE, "golden", "fixtures.npz"))
    return f, json.loads(str(f["meta"]))


def act(seed, stream, n):
    bits = O.synth_normal_array(seed, stream, 0, n, 1.0, O.BF16)
    return bits, O.to_f32(bits, O.BF16)


def int4_page(spec, k, m, g, sdt):
    seed, stream, sigma = spec
    return O.synth_int4_page(seed, stream, k, g, sdt, sigma, 0, m)


def test_gemv_fixtures():
    f, meta = load()
    for name in ("gemv_bf16_g32", "gemv_f16_g128"):
        m = meta[name]
        page = int4_page(m["page"], m["k"], m["m"], m["g"], m["scale_dt"])
        _, x = act(m["x"][0], m["x"][1], m["k"])
        assert np.array_equal(O.matmul_int4_acc(x, page, m["k"], m["m"], m["g"], m["scale_dt"]),
                              f[name])


def test_swiglu_fixture():
    f, meta = load()
    m = meta["swiglu_bf16_g32"]
    up = int4_page(m["up"], m["k"], m["m"], m["g"], m["scale_dt"])
    gate = int4_page(m["gate"], m["k"], m["m"], m["g"], m["scale_dt"])
    _, x = act(m["x"][0], m["x"][1], m["k"])
    h = O.swiglu_int4_acc(x, up, gate, m["k"], m["m"], m["g"], m["scale_dt"])
    assert np.array_equal(h, f["swiglu_bf16_g32"])


def test_router_fixture():
    f, meta = load()
    m = meta["router"]
    w = O.synth_normal_array(m["w"][0], m["w"][1], 0, m["E"] * m["D"], m["w"][2], O.F32)
    b = O.synth_normal_array(m["bias"][0], m["bias"][1], 0, m["E"], m["bias"][2], O.F32)
    _, x = act(m["x"][0], m["x"][1], m["D"])
    ids, wts, scores = O.router(x, w, O.F32, m["E"], m["D"], m["top_k"], m["mode"], m["scaling"],
                                bool(m["normalize"]), b)
    assert [int(i) for i in ids] == list(f["router_ids"])
    assert np.array_equal(wts, f["router_wts"]) and np.array_equal(scores, f["router_scores"])


def layer_pages(seed, hidden, inter, g, sdt, sigma, n):
    return {e: [O.synth_int4_page(seed, 100 + 3 * e + s, *((hidden, g) if s < 2 else (inter, g)),
                                  sdt, sigma, 0, inter if s < 2 else hidden) for s in range(3)]
            for e in range(n)}


def test_layer_fixture():
    f, meta = load()
    m = meta["layer"]
    seed = m["x"][0]
    pages = layer_pages(seed, m["hidden"], m["inter"], m["g"], m["scale_dt"], m["sigma"],
                        m["experts"])
    _, x = act(seed, m["x"][1], m["hidden"])
    rows = [m["inter"], m["inter"], m["hidden"]]
    ids = f["layer_ids"].astype(np.uint16)
    routed = {int(e): ([[p] for p in pages[int(e)]], rows) for e in ids}
    shared = [([[p] for p in pages[s]], rows) for s in m["shared"]]
    out = O.moe_layer(x, m["hidden"], m["inter"], m["g"], m["scale_dt"], routed, ids,
                      f["layer_wts"], shared, faithful=True)
    assert np.array_equal(out, f["layer_out"])


def mxfp4_pages(seed, hidden, inter, n):
    return [tuple(O.synth_mxfp4_page(seed, 200 + 3 * e + s,
                                     *((hidden, 0, inter) if s < 2 else (inter, 0, hidden)))
                  for s in range(3)) for e in range(n)]


def test_mxfp4_fixture():
    f, meta = load()
    m = meta["mxfp4"]
    seed = m["x"][0]
    pages = mxfp4_pages(seed, m["hidden"], m["inter"], m["E"])
    _, x = act(seed, m["x"][1], m["tokens"] * m["hidden"])
    out = O.moe_mxfp4_batched(x.reshape(m["tokens"], m["hidden"]), m["hidden"], m["inter"], pages,
                              f["mxfp4_ids"].astype(np.uint16), f["mxfp4_wts"])
    assert np.array_equal(out, f["mxfp4_out_bf16"])


def test_rmsnorm_fixture():
    f, meta = load()
    m = meta["rmsnorm"]
    seed, stream, sigma = m["x"]
    x = O.synth_normal_array(seed, stream, 0, m["n"], sigma, O.F32)
    wseed, wstream, wsigma, woff = m["w"]
    w = (O.synth_normal_array(wseed, wstream, 0, m["n"], wsigma, O.F32) + np.float32(woff)).astype(
        np.float16)
    y = O.rms_norm_f32(x, w.view(np.uint16), m["eps"])
    assert np.array_equal(y, f["rmsnorm_out"])
    gseed, gstream, gsigma = m["gate"]
    gw = O.synth_normal_array(gseed, gstream, 0, m["n"], gsigma, O.F16)
    assert np.float32(O.sigmoid(O.linear_row_f16(y, gw))) == f["rmsnorm_gate"][0]
