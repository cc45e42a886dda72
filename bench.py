"""Benchmark: MoE layer decode (batch 1, Kimi-K2.5 shape) on one MI355X.

A step = one full MoE sublayer decode for one token over experts resident in HBM: router
(384 experts, fp32 weights, sigmoid + bias, top-8, normalised, x2.827) -> fused INT4 gate/up GEMV
+ SwiGLU over the 8 routed + 1 shared experts -> INT4 down GEMV with the weighted expert sum.
Workload = BASELINE.json configs[2] (c2); --config c3 runs the paged variant (64-row tiles at
shuffled offsets of a 16 GB pool), --config c1 the Mixtral-shape layer.

Every step uses a different token and the steps rotate over `--layers` independent layers
(separate router and expert weights), so the weights a step reads were last touched
>= layers * 234 MB earlier and are not served from the 256 MB last-level cache: the timed
bytes come from HBM, as in a real decode that walks through 61 layers.

Before the W counted warm-up steps, the bench runs steps for `--settle-ms` (200 ms) of wall
time: the GPU comes to the benchmark idle and needs ~0.1 s of load to leave its low clock
state (with 5 warm-up steps alone, the first timed steps ran ~3 us per layer slower). The line
reports how many settle steps ran, and per-step median / p90 / max from a separate pass.

Prints ONE JSON line (rank 0). `value` = microseconds per layer (lower is better).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

CONFIGS = {
    "c2": dict(workload="c2: Kimi-K2.5 MoE layer decode, batch 1 (router fp32 [384,7168] sigmoid+bias "
                        "top-8 x2.827 normalised; 8 routed + 1 shared INT4 experts, hidden 7168, "
                        "inter 2048, g32 bf16 scales; x bf16)",
               hidden=7168, inter=2048, g=32, sdt="bf16", sigma=0.01, E=384, shared=1, k=8,
               mode=1, scaling=2.827, router_sigma=0.01, bias_sigma=0.1, x_dtype="bf16",
               layout="contiguous", seed=0x5EED0002, layers=8),
    "c3": dict(workload="c3: c2 paged into 64-row INT4 tiles at shuffled offsets of a 16 GB pool",
               hidden=7168, inter=2048, g=32, sdt="bf16", sigma=0.01, E=384, shared=1, k=8,
               mode=1, scaling=2.827, router_sigma=0.01, bias_sigma=0.1, x_dtype="bf16",
               layout="paged", seed=0x5EED0003, layers=4),
    "c4": dict(workload="c4: batched decode, 64 tokens bf16, top-8 Zipf(1.1) over 384 MXFP4 experts "
                        "(Kimi-K2.5 shape: hidden 7168, inter 2048; e2m1 codes, e8m0 per 32), "
                        "grouped per expert as a grouped GEMM on MFMA with fused SwiGLU, bf16 out",
               hidden=7168, inter=2048, E=384, k=8, tokens=64, zipf=1.1, seed=0x5EED0004,
               layers=2, batches=8),
    "fp4": dict(workload="reference fused NVFP4 MoE (vib3_launch_moe_experts_fused_gpu, "
                         "kernels.cu:5868) at Kimi-K2.5 shape: FP4 activation quantize + 8 of "
                         "384 experts (tiled split-half E2M1, bf16-exponent scales per 32), "
                         "hidden 7168, inter 2048, device page table u64[L][E][3]",
                hidden=7168, inter=2048, E=384, k=8, seed=0x5EED0005, layers=4),
    "c1": dict(workload="c1: Mixtral-8x7B MoE layer decode, batch 1 (router fp32 [8,4096] softmax "
                        "top-2; 8 INT4 experts 14336x4096, g128 fp16 scales; x fp16)",
               hidden=4096, inter=14336, g=128, sdt="f16", sigma=0.02, E=8, shared=0, k=2,
               mode=0, scaling=1.0, router_sigma=0.02, bias_sigma=None, x_dtype="f16",
               layout="contiguous", seed=0x5EED0001, layers=4),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def algorithmic_bytes(cfg, shape) -> dict:
    """Bytes the decode must read: touched experts' pages, router weights + bias, activation."""
    from vib3_amd.moe import page_bytes
    gu = 2 * page_bytes(cfg["inter"], cfg["hidden"], cfg["g"])
    dn = page_bytes(cfg["hidden"], cfg["inter"], cfg["g"])
    n = cfg["k"] + cfg["shared"]
    x_bytes = cfg["hidden"] * (2 if cfg["x_dtype"] != "f32" else 4)
    router = cfg["E"] * cfg["hidden"] * 4 + (cfg["E"] * 4 if cfg["bias_sigma"] is not None else 0)
    h_bytes = n * cfg["inter"] * 2
    return {
        "router": router + x_bytes,
        "gateup": n * gu + x_bytes + h_bytes,          # weights + x in, h out
        "down": n * dn + h_bytes + cfg["hidden"] * 4,  # weights + h in, out
        "layer": router + n * (gu + dn) + x_bytes + cfg["hidden"] * 4,
    }


def host_cpu() -> dict:
    """The CPU the baseline runs on: model, logical CPUs, the CPUs this process may use, and
    the threads the baseline uses (this pool gives each GPU's process a 16-CPU share)."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                         None)
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or affinity
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": affinity,
            "threads": max(1, min(affinity, share))}


def median_time(fn, budget_s: float, min_reps: int = 3, max_reps: int = 200):
    """Median wall time of fn() over about budget_s seconds (after one warm-up call)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_reps:
            break
    return statistics.median(times), len(times)


def settle(step, ms: float, sync) -> int:
    """Run `step` back to back for about `ms` milliseconds of wall time before the counted
    warm-up: a GPU that has been idle (the bench's setup ends in host work) starts at low
    clocks and needs ~0.1 s of load to reach its steady state; a decode loop runs
    continuously. Returns the number of steps run."""
    n, t_end = 0, time.perf_counter() + ms / 1e3
    while time.perf_counter() < t_end:
        for _ in range(50):
            step(n)
            n += 1
        sync()
    return n


def per_step_stats(step, first: int, k: int, stream) -> dict:
    """Median / p90 / max of single steps, each bracketed by its own pair of HIP events on the
    launch stream (a separate pass after the timed region; the events add a little time)."""
    from vib3_amd import _hip
    k = max(1, min(k, 500))
    ev = [(_hip.Event(), _hip.Event()) for _ in range(k)]
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        step(first + i)
        b.record(stream)
    ev[-1][1].synchronize()
    us = sorted(a.elapsed_ms(b) * 1e3 for a, b in ev)
    return {"median": round(statistics.median(us), 3),
            "p90": round(us[min(len(us) - 1, int(0.9 * len(us)))], 3),
            "max": round(us[-1], 3), "steps": k}


def cpu_baseline(cfg, bank, w, b, x, ids, wts, budget_s: float):
    """Time the oracle (C restatement of vib3's CPU fallback) on the same layer and token, with
    every thread of the process's CPU share and with one thread."""
    import numpy as np
    from oracle import oracle as O
    host = host_cpu()
    threads = host["threads"]
    xh = x.float().cpu().numpy()
    wh = w.cpu().numpy()
    bh = b.cpu().numpy() if b is not None else None
    ids = ids.astype(np.uint16)
    routed = {int(e): bank.expert_pages_host(int(e)) for e in ids}
    shared = [bank.expert_pages_host(cfg["E"] + s) for s in range(cfg["shared"])]
    sdt = O.BF16 if cfg["sdt"] == "bf16" else O.F16

    def one(n):
        r_ids, r_wts, _ = O.router(xh, wh, O.F32, cfg["E"], cfg["hidden"], cfg["k"], cfg["mode"],
                                   cfg["scaling"], True, bh, nthreads=n)
        O.moe_layer(xh, cfg["hidden"], cfg["inter"], cfg["g"], sdt, routed, r_ids, r_wts, shared,
                    faithful=True, nthreads=n)

    med, reps = median_time(lambda: one(threads), budget_s)
    med1, reps1 = median_time(lambda: one(1), budget_s / 2, min_reps=3, max_reps=50)
    return {"value": med * 1e6, "unit": "us/layer", "cores": threads, "kind": "port",
            "single_thread_us": round(med1 * 1e6, 1), "host": host,
            "sample": f"c-oracle restatement of kernels.rs CPU fallback (router + "
                      f"{cfg['k']}+{cfg['shared']} experts, f16 rounding points kept) on the same "
                      f"layer/token as the GPU; median of {reps} reps with {threads} threads (the "
                      f"process's CPU share), median of {reps1} reps with 1 thread",
            "reps": reps}


def bench_c4(args, cfg) -> int:
    """c4: batched MXFP4 decode. A step = one batch of 64 tokens through the MoE sublayer."""
    import numpy as np
    import torch

    from vib3_amd import _hip, _lib, mxfp4

    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    H, I, E, K, T = cfg["hidden"], cfg["inter"], cfg["E"], cfg["k"], cfg["tokens"]
    L = args.layers or cfg["layers"]
    t0 = time.perf_counter()
    banks = []
    for l in range(L):
        banks.append(mxfp4.Mxfp4ExpertBank(H, I, E, layer=l, seed=cfg["seed"], device=dev))
        torch.cuda.synchronize()
        log(f"[bench] layer {l} ready ({banks[-1].nbytes / 1e9:.2f} GB, {time.perf_counter() - t0:.1f}s)")
    nb = cfg["batches"]
    picks = [mxfp4.zipf_picks(T, E, K, s=cfg["zipf"], seed=cfg["seed"] + b) for b in range(nb)]
    xs = []
    for b in range(nb):
        x = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
        _lib.call("vib3_synth_normal", x.data_ptr(), 2, T * H, cfg["seed"], 1000 + b, 0, 1.0, st)
        xs.append(x)
    dev_picks = [(torch.from_numpy(i.view(np.int16)).to(dev), torch.from_numpy(w).to(dev))
                 for i, w in picks]
    runners = [mxfp4.MoeMxfp4Batch(bk, T, K) for bk in banks]
    descs = [[r.desc(xs[b], *dev_picks[b]) for b in range(nb)] for r in runners]
    launch = _lib.load().vib3_launch_moe_mxfp4_batched

    def step(i):
        rc = launch(descs[i % L][i % nb], st)
        if rc:
            raise _lib.Vib3Error("vib3_launch_moe_mxfp4_batched", rc)

    n_settle = settle(step, args.settle_ms, torch.cuda.synchronize)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = _hip.Event(), _hip.Event()
    e0.record(st)
    for i in range(args.steps):
        step(args.warmup + i)
    e1.record(st)
    e1.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / args.steps
    step_stats = per_step_stats(step, args.warmup + args.steps, args.steps, st)

    # algorithmic bytes: every touched expert's three pages once, activations in, output out
    ebytes = banks[0].expert_bytes
    distinct = [len(np.unique(i)) for i, _ in picks]
    avg_bytes = float(np.mean(distinct)) * ebytes + 2 * T * H * 2
    flops = T * K * 3 * 2 * H * I
    gbs = avg_bytes / (us * 1e-6) / 1e9
    log(f"[bench] {args.steps} batches: {us:.1f} us/batch, {np.mean(distinct):.1f} experts/batch, "
        f"{gbs:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        ids, w = picks[0]
        xh = O.to_f32(xs[0].view(torch.int16).cpu().numpy().view(np.uint16).ravel(),
                      O.BF16).reshape(T, H)
        used = sorted({int(e) for e in ids.ravel()})
        empty = np.zeros(1, dtype=np.uint8)
        pages = [banks[0].expert_pages_host(e) if e in used else (empty, empty, empty)
                 for e in range(E)]
        host = host_cpu()
        threads = host["threads"]
        # the whole 64-token batch 0 with the process's CPU share (one warm-up, then timed runs
        # within the budget, at least one)
        full, reps = median_time(
            lambda: O.moe_mxfp4_batched(xh, H, I, pages, ids, w, nthreads=threads),
            args.cpu_seconds, min_reps=1, max_reps=5)
        # one thread: token 0 alone, stated as such
        one, reps1 = median_time(
            lambda: O.moe_mxfp4_batched(xh[:1], H, I, pages, ids[:1], w[:1], nthreads=1),
            args.cpu_seconds / 2, min_reps=2, max_reps=20)
        cpu = {"value": round(full * 1e6, 1), "unit": "us/batch", "cores": threads,
               "kind": "port", "host": host,
               "single_thread_us_per_token": round(one * 1e6, 1),
               "sample": f"c-oracle per-token restatement over all {T} tokens of batch 0 "
                         f"(8 experts each, {len(used)} distinct), median of {reps} runs with "
                         f"{threads} threads; single thread: token 0, median of {reps1} runs"}

    traffic = None  # HBM bytes per batch of the two GEMM launches, from the committed PMC summary
    tpath = os.path.join(ROOT, "profiles", "traffic_c4.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            kern = json.load(f)["kernels"]
        traffic = sum(kern[k]["hbm_bytes"] for k in kern)
    out = {
        "metric": "MoE batched decode us per 64-token batch (Kimi-K2.5 shape, MXFP4 experts)",
        "value": round(us, 2), "unit": "us/batch", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4 weights x bf16 activations, bf16/f16 MFMA, f32 accumulate",
        "data": "synthetic (counter-based generator; random-init weights of the named shape)",
        "config": {"workload": cfg["workload"], "layers_rotated": L, "batches": nb,
                   "distinct_experts_per_batch": round(float(np.mean(distinct)), 1),
                   "algorithmic_bytes_per_batch": round(avg_bytes)},
        "roofline": {"bound": "hbm", "kernel": "k_mx_rows + k_mx_gemm (row path and matrix-core grouped GEMM, gate/up + down, whole batch)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": "profiles/traffic_c4.json" if traffic else None},
        "mfma": {"achieved_tflops": round(flops / (us * 1e-6) / 1e12, 2), "peak_tflops_bf16": 2500.0,
                 "frac": round(flops / (us * 1e-6) / 2.5e15, 5)},
        "tokens_per_s": round(T / (us * 1e-6)),
        "per_step_us": step_stats,
        "settle": {"ms": args.settle_ms, "steps": n_settle},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def given_ids_pass(layers, xs, cfg, args, lib, st, nbytes) -> dict:
    """The same layers with the experts given as ids (seeded picks, no router): the path the
    reference engine takes after its own router launch, so the expert GEMVs run without the
    routing window that the fused gate/up kernel spends computing and polling the logits.
    Reported beside the headline, which is the fused layer; the roofline stays on the fused
    kernel."""
    import numpy as np
    import torch

    from vib3_amd import _hip, _lib

    dev = xs[0].device
    rng = np.random.default_rng(cfg["seed"] + 1)
    gid = [torch.from_numpy(rng.choice(cfg["E"], cfg["k"], replace=False).astype(np.int16)).to(dev)
           for _ in range(args.tokens)]
    gw = torch.full((cfg["k"],), 1.0 / cfg["k"], dtype=torch.float32, device=dev)
    descs = []
    for ly in layers:
        row = []
        for t, x in enumerate(xs):
            d = ly._desc(x, gid[t], gw)
            d.router_w = None
            row.append(d)
        descs.append(row)
    L = len(layers)
    stage = {}
    for j, name in ((1, "gateup"), (2, "down")):
        for i in range(args.warmup):
            lib.vib3_launch_moe_int4_layer(descs[i % L][i % args.tokens], st)
        s0, s1 = _hip.Event(), _hip.Event()
        s0.record(st)
        for i in range(args.steps):
            d = descs[i % L][i % args.tokens]
            rc = lib.vib3_launch_moe_int4_layer_stage(d, j, st)
            if rc:
                raise _lib.Vib3Error("vib3_launch_moe_int4_layer_stage", rc)
        s1.record(st)
        s1.synchronize()
        stage[name] = s0.elapsed_ms(s1) * 1e3 / args.steps
    gu = nbytes["gateup"] / (stage["gateup"] * 1e-6) / 1e9
    both = (nbytes["gateup"] + nbytes["down"]) / ((stage["gateup"] + stage["down"]) * 1e-6) / 1e9
    return {"stages_us": {k: round(v, 3) for k, v in stage.items()},
            "gateup_gbs": round(gu, 1), "gateup_frac": round(gu / HBM_PEAK_GBS, 4),
            "gemv_gbs": round(both, 1), "gemv_frac": round(both / HBM_PEAK_GBS, 4),
            "note": "seeded ids given (no router): the expert GEMV kernels alone"}


def bench_fp4(args, cfg) -> int:
    """The reference's sync-free fused NVFP4 path: a step = quantize the f32 activation to FP4
    + vib3_launch_moe_experts_fused_gpu over 8 experts of a 384-expert layer (the launches the
    engine issues per MoE layer, engine.rs:5143-5179)."""
    import numpy as np
    import torch

    from vib3_amd import _hip, _lib

    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    H, I, E, K = cfg["hidden"], cfg["inter"], cfg["E"], cfg["k"]
    L = args.layers or cfg["layers"]
    g = torch.Generator(device=dev).manual_seed(cfg["seed"])
    data_gu, data_dn = H // 2 * I, I // 2 * H
    sc_gu, sc_dn = I * (H // 32) * 2, H * (I // 32) * 2
    page = [data_gu + sc_gu, data_gu + sc_gu, data_dn + sc_dn]
    ebytes = sum(page)
    t0 = time.perf_counter()
    pools, table = [], np.zeros((L, E, 3), dtype=np.uint64)
    for l in range(L):
        pool = torch.randint(0, 256, (E * ebytes,), dtype=torch.uint8, device=dev, generator=g)
        base = pool.data_ptr()
        per_e = pool.view(E, ebytes)
        off = 0
        for s in range(3):  # bf16 scales: exponent 119..123 (2^-8..2^-4), random mantissa
            rows, k = (I, H) if s < 2 else (H, I)
            table[l, :, s] = base + np.arange(E, dtype=np.uint64) * ebytes + off
            sc = per_e[:, off + rows * k // 2: off + page[s]].view(torch.int16)
            ex = torch.randint(119, 124, sc.shape, dtype=torch.int16, device=dev, generator=g)
            sc.copy_((ex << 7) | (sc & 0x7F))
            off += page[s]
        pools.append(pool)
        torch.cuda.synchronize()
        log(f"[bench] fp4 layer {l} ready ({pool.numel() / 1e9:.2f} GB, {time.perf_counter() - t0:.1f}s)")
    tab = torch.from_numpy(table.view(np.int64)).to(dev)
    rng = np.random.default_rng(cfg["seed"])
    T = args.tokens
    xs = [torch.randn(H, dtype=torch.float32, device=dev, generator=g) for _ in range(T)]
    ids = [torch.from_numpy(rng.choice(E, K, replace=False).astype(np.int16)).to(dev)
           for _ in range(T)]
    wts = torch.full((K,), 1.0 / K, dtype=torch.float32, device=dev)
    codes = torch.zeros(H // 2, dtype=torch.uint8, device=dev)
    scs = torch.zeros(H // 32, dtype=torch.uint8, device=dev)
    out = torch.zeros(H, dtype=torch.float32, device=dev)
    lib = _lib.load()
    _lib.call("vib3_moe_prewarm_gpu_bufs", I, I)

    def step(i):
        rc = lib.vib3_launch_quantize_activation_fp4(xs[i % T].data_ptr(), codes.data_ptr(),
                                                     scs.data_ptr(), H, st)
        rc = rc or lib.vib3_launch_moe_experts_fused_gpu(
            codes.data_ptr(), scs.data_ptr(), tab.data_ptr(), ids[i % T].data_ptr(),
            wts.data_ptr(), i % L, E, K, H, I, I, H, out.data_ptr(), st)
        if rc:
            raise _lib.Vib3Error("fp4 fused step", rc)

    n_settle = settle(step, args.settle_ms, torch.cuda.synchronize)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = _hip.Event(), _hip.Event()
    e0.record(st)
    for i in range(args.steps):
        step(args.warmup + i)
    e1.record(st)
    e1.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / args.steps
    step_stats = per_step_stats(step, args.warmup + args.steps, args.steps, st)
    nbytes = K * ebytes + H * 4 + H // 2 + H // 32 + 2 * H * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"[bench] fp4 fused: {us:.2f} us/layer, {gbs:.0f} GB/s")
    traffic = None  # HBM bytes per step of the three launches, from the committed PMC summary
    tpath = os.path.join(ROOT, "profiles", "traffic_fp4.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = sum(v["hbm_bytes"] for v in json.load(f)["kernels"].values())
    out_line = {
        "metric": "fused NVFP4 MoE layer decode us (batch 1, Kimi-K2.5 shape)",
        "value": round(us, 3), "unit": "us/layer", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "e2m1 weights x e2m1 activations, exact group sums, f64/f32 accumulate",
        "data": "synthetic (random codes, bf16 scales of exponent 2^-8..2^-4)",
        "config": {"workload": cfg["workload"], "layers_rotated": L, "tokens": T,
                   "algorithmic_bytes_per_layer": nbytes},
        "roofline": {"bound": "hbm", "kernel": "k_fp4_quant_act + k_fp4_gateup + k_fp4_down (whole step)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": "profiles/traffic_fp4.json" if traffic else None},
        "cpu_baseline": None,
        "per_step_us": step_stats,
        "settle": {"ms": args.settle_ms, "steps": n_settle},
    }
    print(json.dumps(out_line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=0, help="layers to rotate (default per config)")
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed steps before the warm-up, until the GPU clocks settle "
                         "(0: none; the number is reported)")
    ap.add_argument("--sublayer", action="store_true",
                    help="the whole MoE sublayer as the engine runs it: x is the f32 residual "
                         "stream, RMSNorm + shared-expert sigmoid gate + residual add fused in")
    ap.add_argument("--given-ids", action="store_true",
                    help="skip the router: experts come from preset device id lists (diagnostic)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build targets a single MI355X (no multi-GPU "
              "path); run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from vib3_amd import _hip, _lib, moe
    from vib3_amd._lib import DT_BF16, DT_F16, DT_F32

    cfg = dict(CONFIGS[args.config])
    if args.config == "c4":
        return bench_c4(args, cfg)
    if args.config == "fp4":
        return bench_fp4(args, cfg)
    if args.layers:
        cfg["layers"] = args.layers
    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[cfg["x_dtype"]]
    shape = moe.BankShape(hidden=cfg["hidden"], inter=cfg["inter"], group_size=cfg["g"],
                          scale_dtype=DT_BF16 if cfg["sdt"] == "bf16" else DT_F16,
                          scale_sigma=cfg["sigma"], num_experts=cfg["E"], num_shared=cfg["shared"])

    t0 = time.perf_counter()
    layers = []
    for l in range(cfg["layers"]):
        bank = moe.Int4ExpertBank(shape, layer=l, seed=cfg["seed"], layout=cfg["layout"],
                                  tile_rows=64, pool_bytes=(16 << 30) if cfg["layout"] == "paged" else None,
                                  device=dev)
        w, b = moe.make_router(shape, l, cfg["seed"], cfg["router_sigma"], cfg["bias_sigma"],
                               device=dev)
        extra = {}
        if args.sublayer:
            g = torch.Generator(device="cpu").manual_seed(cfg["seed"] + l)
            extra = dict(
                norm_weight=(1 + 0.1 * torch.randn(cfg["hidden"], generator=g)).half().to(dev),
                norm_eps=1e-6,
                shared_gate=(0.02 * torch.randn(cfg["shared"], cfg["hidden"], generator=g))
                .half().to(dev) if cfg["shared"] else None)
        layers.append(moe.MoeInt4Layer(bank, w, b, top_k=cfg["k"], scoring_mode=cfg["mode"],
                                       scaling_factor=cfg["scaling"], normalize=True, **extra))
        torch.cuda.synchronize()
        log(f"[bench] layer {l} ready ({bank.nbytes / 1e9:.2f} GB, {time.perf_counter() - t0:.1f}s)")
    if args.sublayer:  # the residual stream between decoder layers: f32, large magnitudes
        tdt = torch.float32
    xs = [moe.make_activation(cfg["hidden"], t, cfg["seed"], dtype=tdt, device=dev)
          for t in range(args.tokens)]
    if args.sublayer:
        xs = [x * 20.0 for x in xs]
    if args.given_ids:
        rng = np.random.default_rng(cfg["seed"])
        gid = [torch.from_numpy(rng.choice(cfg["E"], cfg["k"], replace=False).astype(np.int16)).to(dev)
               for _ in range(args.tokens)]
        gw = torch.full((cfg["k"],), 1.0 / cfg["k"], dtype=torch.float32, device=dev)
        for ly in layers:
            ly.router_w = None
        descs = [[ly._desc(x, gid[t], gw) for t, x in enumerate(xs)] for ly in layers]
    else:
        descs = [[ly._desc(x) for x in xs] for ly in layers]
    if args.sublayer:  # out = x + MoE(RMSNorm(x)), engine.rs:5064-5307
        for row in descs:
            for d, x in zip(row, xs):
                d.residual = x.data_ptr()
    lib = _lib.load()
    launch = lib.vib3_launch_moe_int4_layer
    L = len(layers)

    def step(i: int) -> None:
        rc = launch(descs[i % L][i % args.tokens], st)
        if rc:
            raise _lib.Vib3Error("vib3_launch_moe_int4_layer", rc)

    n_settle = settle(lambda i: step(i), args.settle_ms, torch.cuda.synchronize)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = _hip.Event(), _hip.Event()
    torch.cuda.synchronize()
    e0.record(st)
    for i in range(args.steps):
        step(args.warmup + i)
    e1.record(st)
    e1.synchronize()
    torch.cuda.synchronize()
    total_ms = e0.elapsed_ms(e1)
    us_per_layer = total_ms * 1e3 / args.steps
    log(f"[bench] {args.steps} steps: {us_per_layer:.2f} us/layer (after {n_settle} settle steps)")
    step_stats = per_step_stats(step, args.warmup + args.steps, args.steps, st)

    # per-stage times: each stage's launches alone, back to back over the same rotation of
    # layers and tokens (a stage reads what the full-layer launches above left in its workspace)
    fused = bool(lib.vib3_moe_int4_router_fused(descs[0][0]))
    stage_us = {}
    for j, name in enumerate(("router", "gateup", "down")):
        if name == "router" and args.sublayer and fused:
            name = "prologue"  # RMSNorm + shared gates; the router is inside gate/up
        elif name == "router" and (args.given_ids or fused):
            continue  # no router launches: the gate/up kernel computes the logits itself
        s0, s1 = _hip.Event(), _hip.Event()
        s0.record(st)
        for i in range(args.steps):
            rc = lib.vib3_launch_moe_int4_layer_stage(descs[i % L][(args.warmup + i) % args.tokens],
                                                      j, st)
            if rc:
                raise _lib.Vib3Error("vib3_launch_moe_int4_layer_stage", rc)
        s1.record(st)
        s1.synchronize()
        stage_us[name] = s0.elapsed_ms(s1) * 1e3 / args.steps

    nbytes = algorithmic_bytes(cfg, shape)
    given = None
    if fused and not args.sublayer:
        given = given_ids_pass(layers, xs, cfg, args, lib, st, nbytes)
    if fused:  # the gate/up kernel also reads the router weights
        nbytes["gateup"] += nbytes["router"]
    gu_gbs = nbytes["gateup"] / (stage_us["gateup"] * 1e-6) / 1e9
    layer_gbs = nbytes["layer"] / (us_per_layer * 1e-6) / 1e9
    expert_gbs = (nbytes["gateup"] + nbytes["down"]) / ((stage_us["gateup"] + stage_us["down"]) * 1e-6) / 1e9

    copy_gbs = None
    if True:  # achievable device copy bandwidth, reported beside the 8 TB/s peak
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device=dev)
        dst = torch.empty(n, dtype=torch.uint8, device=dev)
        dst.copy_(src)
        torch.cuda.synchronize()
        c0, c1 = _hip.Event(), _hip.Event()
        c0.record(st)
        for _ in range(10):
            dst.copy_(src)
        c1.record(st)
        c1.synchronize()
        copy_gbs = 2 * n * 10 / (c0.elapsed_ms(c1) * 1e-3) / 1e9
        del src, dst

    # HBM traffic per launch of the roofline kernel, from the committed rocprofv3 PMC summary
    # (FETCH_SIZE + WRITE_SIZE, each scaled by what the counter reads for a 1 GiB copy)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tpath) and not args.given_ids:
        with open(tpath) as f:
            kern = json.load(f)["kernels"]
            traffic = next((v["hbm_bytes"] for k, v in kern.items()
                            if k.startswith("k_int4_rows")), None)

    cpu = None
    if not args.no_cpu and not args.given_ids and not args.sublayer:
        ly = layers[0]
        x = xs[0]
        ly.launch(x)
        torch.cuda.synchronize()
        ids = ly.ids.cpu().numpy().view(np.uint16)[: cfg["k"]]
        wts = ly.wts.cpu().numpy()[: cfg["k"]]
        cpu = cpu_baseline(cfg, ly.bank, ly.router_w, ly.router_bias, x, ids, wts,
                           args.cpu_seconds)
        log(f"[bench] cpu baseline {cpu['value']:.0f} us/layer ({cpu['cores']} threads)")

    out = {
        "metric": "MoE layer decode us (batch 1, Kimi-K2.5 shape); expert GEMV achieved HBM GB/s"
                  if args.config != "c1" else "MoE layer decode us (batch 1, Mixtral shape)",
        "value": round(us_per_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"int4 weights x {'f32' if args.sublayer else cfg['x_dtype']} activations, "
                 "f32 accumulate",
        "data": "synthetic (counter-based generator; random-init weights of the named shape)",
        "config": {"workload": cfg["workload"] + ("; whole sublayer: f32 residual stream in, "
                                                  "RMSNorm, sigmoid-gated shared expert, "
                                                  "residual add" if args.sublayer else ""),
                   "layers_rotated": L, "tokens": args.tokens,
                   "layout": cfg["layout"], "algorithmic_bytes_per_layer": nbytes["layer"]},
        "roofline": {"bound": "hbm",
                     "kernel": "k_int4_rows (router logits + top-k + gate/up GEMV + SwiGLU)"
                               if fused else "k_int4_rows (top-k + gate/up GEMV + SwiGLU)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": f"profiles/traffic_{args.config}.json" if traffic else None,
                     "algorithmic_bytes_per_launch": nbytes["gateup"],
                     "avg_launch_us": round(stage_us["gateup"], 3)},
        "stages_us": {k: round(v, 3) for k, v in stage_us.items()},
        "per_step_us": step_stats,
        "settle": {"ms": args.settle_ms, "steps": n_settle},
        "layer_gbs": round(layer_gbs, 1),
        "expert_gemv_gbs": round(expert_gbs, 1),
        "expert_gemv_given_ids": given,
        "copy_gbs": round(copy_gbs, 1) if copy_gbs else None,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
