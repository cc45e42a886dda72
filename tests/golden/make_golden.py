"""Write tests/golden/fixtures.npz: small known-answer cases for the INT4 GEMV, the fused SwiGLU,
the router top-k, a small MoE layer, a batched MXFP4 MoE, and the pre-MoE RMSNorm with the
shared expert's sigmoid gate.

Inputs are not stored: they come from the counter-based generator (seed, stream) shared by the
oracle (oracle/cpu_ref.c) and the device (vib3_amd/csrc/synth.hip), so a fixture holds the
generator parameters and the expected outputs. The expected outputs are the oracle's, and this
script refuses to write them unless an independent float64 recomputation (numpy) agrees.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.npz")
SEED = 0x601D


def dense_int4(page, rows, k, g, sdt):
    """float64 dense matrix of an INT4 page (numpy only)."""
    pk, ng = (k + 1) // 2, (k + g - 1) // g
    codes = page[: rows * pk].reshape(rows, pk)
    q = np.empty((rows, 2 * pk), dtype=np.int64)
    q[:, 0::2] = codes & 15
    q[:, 1::2] = codes >> 4
    sb = page[rows * pk: rows * pk + rows * ng * 2].view(np.uint16).reshape(rows, ng)
    if sdt == O.BF16:
        s = (sb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    else:
        s = sb.view(np.float16).astype(np.float64)
    s = np.where(np.isfinite(s) & (s > 0), s, 0.125)
    return (q[:, :k] - 8) * np.repeat(s, g, axis=1)[:, :k]


def dense_mx(page, rows, k):
    lut = np.array([(-1.0 if c & 8 else 1.0) * [0, 0.5, 1, 1.5, 2, 3, 4, 6][c & 7]
                    for c in range(16)])
    codes = page[: rows * k // 2].reshape(rows, k // 2)
    sc = page[rows * k // 2: rows * k // 2 + rows * k // 32].reshape(rows, k // 32)
    q = np.empty((rows, k), dtype=np.int64)
    q[:, 0::2] = codes & 15
    q[:, 1::2] = codes >> 4
    return lut[q] * np.repeat(2.0 ** (sc.astype(np.float64) - 127), 32, axis=1)


def act(n, stream, dt=O.BF16):
    bits = O.synth_normal_array(SEED, stream, 0, n, 1.0, dt)
    return bits, (O.to_f32(bits, dt) if dt != O.F32 else bits)


def main() -> None:
    fx = {}
    meta = {}

    # INT4 GEMV, BF16 scales g32 and FP16 scales g128
    for name, k, m, g, sdt in (("gemv_bf16_g32", 512, 64, 32, O.BF16),
                               ("gemv_f16_g128", 1024, 48, 128, O.F16)):
        page = O.synth_int4_page(SEED, 1, k, g, sdt, 0.02, 0, m)
        _, x = act(k, 2)
        acc = O.matmul_int4_acc(x, page, k, m, g, sdt)
        ref = dense_int4(page, m, k, g, sdt) @ x.astype(np.float64)
        assert np.allclose(acc, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max()), name
        fx[name] = acc
        meta[name] = dict(k=k, m=m, g=g, scale_dt=sdt, page=(SEED, 1, 0.02), x=(SEED, 2, "bf16"))

    # fused SwiGLU (up = stream 3, gate = stream 4)
    k, m, g = 512, 64, 32
    up = O.synth_int4_page(SEED, 3, k, g, O.BF16, 0.02, 0, m)
    gate = O.synth_int4_page(SEED, 4, k, g, O.BF16, 0.02, 0, m)
    _, x = act(k, 2)
    h = O.swiglu_int4_acc(x, up, gate, k, m, g, O.BF16)
    u64 = dense_int4(up, m, k, g, O.BF16) @ x
    g64 = dense_int4(gate, m, k, g, O.BF16) @ x
    ref = g64 / (1 + np.exp(-g64)) * u64
    assert np.allclose(h, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    fx["swiglu_bf16_g32"] = h
    meta["swiglu_bf16_g32"] = dict(k=k, m=m, g=g, scale_dt=O.BF16, up=(SEED, 3, 0.02),
                                   gate=(SEED, 4, 0.02), x=(SEED, 2, "bf16"))

    # router: E=384, D=256, f32 W ~ N(0, 0.05), bias ~ N(0, 0.1), sigmoid top-8 x2.827 normalised
    E, D, kk = 384, 256, 8
    w = O.synth_normal_array(SEED, 5, 0, E * D, 0.05, O.F32)
    b = O.synth_normal_array(SEED, 6, 0, E, 0.1, O.F32)
    _, x = act(D, 7)
    ids, wts, scores = O.router(x, w, O.F32, E, D, kk, 1, 2.827, True, b)
    s64 = w.reshape(E, D).astype(np.float64) @ x
    key = 1 / (1 + np.exp(-s64)) + b
    order = np.argsort(-key, kind="stable")
    assert list(order[:kk]) == [int(i) for i in ids]
    sig = 1 / (1 + np.exp(-s64[order[:kk]]))
    assert np.allclose(wts, sig / sig.sum() * 2.827, rtol=1e-5)
    fx["router_ids"], fx["router_wts"], fx["router_scores"] = ids.astype(np.int64), wts, scores
    meta["router"] = dict(E=E, D=D, top_k=kk, mode=1, scaling=2.827, normalize=1,
                          w=(SEED, 5, 0.05, "f32"), bias=(SEED, 6, 0.1), x=(SEED, 7, "bf16"))

    # small MoE layer: hidden 256, inter 128, 4 routed picks + 1 shared, bf16 scales g32
    hidden, inter, g = 256, 128, 32
    pages = {e: [O.synth_int4_page(SEED, 100 + 3 * e + s, *((hidden, g) if s < 2 else (inter, g)),
                                   O.BF16, 0.02, 0, inter if s < 2 else hidden) for s in range(3)]
             for e in range(6)}
    _, x = act(hidden, 8)
    lids = np.array([4, 1, 3, 0], dtype=np.uint16)
    lw = np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float32)
    routed = {int(e): ([[p] for p in pages[int(e)]], [inter, inter, hidden]) for e in lids}
    shared = [([[p] for p in pages[5]], [inter, inter, hidden])]
    out = O.moe_layer(x, hidden, inter, g, O.BF16, routed, lids, lw, shared, faithful=True)
    ref = np.zeros(hidden)
    for e, wv in list(zip(lids, lw)) + [(5, 1.0)]:
        pu, pg, pd = pages[int(e)]
        hu = dense_int4(pu, inter, hidden, g, O.BF16) @ x
        hg = dense_int4(pg, inter, hidden, g, O.BF16) @ x
        hh = (hg / (1 + np.exp(-hg)) * hu).astype(np.float16).astype(np.float64)
        d = (dense_int4(pd, hidden, inter, g, O.BF16) @ hh).astype(np.float16).astype(np.float64)
        ref += float(wv) * d
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-3
    fx["layer_out"] = out
    fx["layer_ids"], fx["layer_wts"] = lids.astype(np.int64), lw
    meta["layer"] = dict(hidden=hidden, inter=inter, g=g, scale_dt=O.BF16, experts=6, shared=[5],
                         page_streams="100 + 3*e + segment (0 up, 1 gate, 2 down)", sigma=0.02,
                         x=(SEED, 8, "bf16"))

    # batched MXFP4 MoE: hidden 256, inter 256, 6 experts, 4 tokens x top-2
    hidden, inter, E, T, k2 = 256, 256, 6, 4, 2
    mx = [tuple(O.synth_mxfp4_page(SEED, 200 + 3 * e + s,
                                   *((hidden, 0, inter) if s < 2 else (inter, 0, hidden)))
                for s in range(3)) for e in range(E)]
    _, xb = act(T * hidden, 9)
    xb = xb.reshape(T, hidden)
    mids = np.array([[0, 3], [5, 0], [2, 2], [1, 4]], dtype=np.uint16)
    mw = np.array([[0.7, 0.3], [0.5, 0.5], [0.6, 0.4], [0.9, 0.1]], dtype=np.float32)
    mout = O.moe_mxfp4_batched(xb, hidden, inter, mx, mids, mw)
    got = O.to_f32(mout.ravel(), O.BF16).reshape(T, hidden)
    ref = np.zeros((T, hidden))
    for t in range(T):
        for j in range(k2):
            e = int(mids[t, j])
            hu = dense_mx(mx[e][0], inter, hidden) @ xb[t]
            hg = dense_mx(mx[e][1], inter, hidden) @ xb[t]
            hh = (hg / (1 + np.exp(-hg)) * hu).astype(np.float16).astype(np.float64)
            d = (dense_mx(mx[e][2], hidden, inter) @ hh).astype(np.float16).astype(np.float64)
            ref[t] += mw[t, j] * d
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-4 * np.abs(ref).max())
    fx["mxfp4_out_bf16"] = mout
    fx["mxfp4_ids"], fx["mxfp4_wts"] = mids.astype(np.int64), mw
    meta["mxfp4"] = dict(hidden=hidden, inter=inter, E=E, tokens=T, top_k=k2,
                         page_streams="200 + 3*e + segment", x=(SEED, 9, "bf16"))

    # pre-MoE RMSNorm (kernels.cu:921) of an f32 residual-stream vector with f16 weights, and
    # the shared expert's sigmoid gate on the result (kernels.rs:3630, kernels.cu:2114)
    n = 1000
    xr = O.synth_normal_array(SEED, 30, 0, n, 20.0, O.F32)
    nw = (O.synth_normal_array(SEED, 31, 0, n, 0.1, O.F32) + np.float32(1.0)).astype(np.float16)
    gw = O.synth_normal_array(SEED, 32, 0, n, 0.02, O.F16)
    y = O.rms_norm_f32(xr, nw.view(np.uint16), 1e-6)
    x64 = xr.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * nw.astype(np.float64)
    assert np.max(np.abs(y - ref)) <= 4e-7 * np.max(np.abs(ref))
    gate = O.sigmoid(O.linear_row_f16(y, gw))
    gref = 1 / (1 + np.exp(-np.dot(y.astype(np.float64), gw.view(np.float16).astype(np.float64))))
    assert abs(gate - gref) <= 1e-6
    fx["rmsnorm_out"] = y
    fx["rmsnorm_gate"] = np.array([gate], dtype=np.float32)
    meta["rmsnorm"] = dict(n=n, eps=1e-6, x=(SEED, 30, 20.0), w=(SEED, 31, 0.1, 1.0),
                           gate=(SEED, 32, 0.02))

    np.savez(OUT, meta=np.array(json.dumps(meta)), **fx)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
