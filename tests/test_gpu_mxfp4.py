"""GPU parity of the batched MXFP4 MoE (vib3_launch_moe_mxfp4_batched) against the CPU oracle.

The oracle restates the batch per token (the reference decodes token by token): h and each
expert output rounded to f16, weighted sum in pick order, bf16 output. The GPU differs only in
the order of f32 additions inside each dot product (matrix-core accumulation for experts with
three or more tokens, a lane-strided GEMV for experts with one or two), so the bar is
rel-L2 <= 1e-3 per token plus: almost every bf16 output equal to the oracle's, out-of-range
picks skipped, repeated launches identical. A token's result depends on the batch only
through which of the two paths each of its experts takes (f32 addition order), so a token
alone and the same token in a batch agree to the same bar, not bit for bit.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 0x5EED0004


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _bank(hidden, inter, E, layer=0):
    from vib3_amd.mxfp4 import Mxfp4ExpertBank
    return Mxfp4ExpertBank(hidden, inter, E, layer=layer, seed=SEED)


def _x(tokens, hidden, stream=77):
    bits = O.synth_normal_array(SEED, stream, 0, tokens * hidden, 1.0, O.BF16)
    host = O.to_f32(bits, O.BF16).reshape(tokens, hidden)
    dev = torch.from_numpy(bits.view(np.int16).reshape(tokens, hidden)).cuda().view(torch.bfloat16)
    return dev, host


def _run(bank, x, ids, w):
    from vib3_amd.mxfp4 import MoeMxfp4Batch
    b = MoeMxfp4Batch(bank, x.shape[0], ids.shape[1])
    out = b.launch(x, torch.from_numpy(ids.view(np.int16)).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy().view(np.uint16).copy()


def _oracle(bank, xh, ids, w, tokens=None):
    E = bank.num_experts
    sel = slice(None) if tokens is None else tokens
    used = sorted({int(e) for e in ids[sel].ravel() if e < E})  # copy back only these
    pages = [bank.expert_pages_host(e) if e in used else None for e in range(E)]
    empty = np.zeros(1, dtype=np.uint8)
    pages = [p if p is not None else (empty, empty, empty) for p in pages]
    return O.moe_mxfp4_batched(xh[sel], bank.hidden, bank.inter, pages, ids[sel], w[sel])


def _check(got_bits, ref_bits):
    got = O.to_f32(got_bits.ravel(), O.BF16).reshape(got_bits.shape)
    ref = O.to_f32(ref_bits.ravel(), O.BF16).reshape(ref_bits.shape)
    for t in range(got.shape[0]):
        r = rel_l2(got[t], ref[t])
        assert r <= 1e-3, (t, r)
    same = float(np.mean(got_bits == ref_bits))
    assert same > 0.97, same
    return same


def test_synth_mxfp4_page_device_matches_oracle():
    from vib3_amd import _lib
    k, rows = 512, 40
    buf = torch.empty(rows * k // 2 + rows * k // 32, dtype=torch.uint8, device="cuda")
    _lib.call("vib3_synth_mxfp4_page", buf.data_ptr(), SEED, 31, k, 8, rows,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(buf.cpu().numpy(), O.synth_mxfp4_page(SEED, 31, k, 8, rows))


@pytest.mark.parametrize("hidden,inter,E,T,k", [(256, 256, 12, 5, 3), (512, 768, 9, 37, 4),
                                                 (256, 256, 3, 70, 2), (2560, 6144, 12, 5, 3),
                                                 (6144, 2560, 6, 9, 2), (4096, 4096, 8, 6, 2),
                                                 (512, 512, 3, 70, 2), (1024, 512, 6, 130, 3)])
def test_small_batches_match_oracle(hidden, inter, E, T, k):
    """Shapes with 1..70+ tokens per expert (row path, several 16-token matrix-core blocks, a
    64-token chunk and a remainder), experts picked twice by one token, experts never picked,
    and reduction lengths that give the row path 1, 2, 3 and 4 chunks per lane. k multiples of
    512 take the LDS-staged matrix-core kernel, the others the registers-only one."""
    _say(f"[mxfp4] small hidden={hidden} inter={inter} E={E} T={T} k={k}")
    from vib3_amd.mxfp4 import zipf_picks
    bank = _bank(hidden, inter, E)
    ids, w = zipf_picks(T, E, k, seed=T)
    if T > 4:
        ids[3, 1] = ids[3, 0]  # the same expert twice for one token
    x, xh = _x(T, hidden)
    got = _run(bank, x, ids, w)
    ref = _oracle(bank, xh, ids, w)
    same = _check(got, ref)
    _say(f"[mxfp4]   bf16 outputs equal to the oracle's: {same:.4f}")


def test_largest_batch():
    """The most picks one launch takes (tokens x top_k = 4096: 512 tokens x 8), every token
    against the oracle on a small shape."""
    _say("[mxfp4] largest batch: 512 tokens x top-8 over 48 experts")
    from vib3_amd.mxfp4 import zipf_picks
    hidden, inter, E, T, k = 256, 256, 48, 512, 8
    bank = _bank(hidden, inter, E, layer=7)
    ids, w = zipf_picks(T, E, k, s=1.1, seed=SEED + 7)
    x, xh = _x(T, hidden, stream=78)
    got = _run(bank, x, ids, w)
    ref = _oracle(bank, xh, ids, w)
    _check(got, ref)


def test_out_of_range_ids_are_skipped():
    _say("[mxfp4] out-of-range ids")
    hidden, inter, E, T, k = 256, 256, 5, 4, 3
    bank = _bank(hidden, inter, E)
    ids = np.array([[0, 1, 2], [E, 3, 4], [4, 4000, 1], [E + 7, E, E]], dtype=np.uint16)
    w = np.full((T, k), 0.5, dtype=np.float32)
    x, xh = _x(T, hidden)
    got = _run(bank, x, ids, w)
    ref = _oracle(bank, xh, ids, w)
    assert np.all(got[3] == 0)  # no valid pick: +0.0
    _check(got[:3], ref[:3])


def test_kimi_shape_batch_zipf():
    """c4: 64 tokens, 384 MXFP4 experts of the Kimi-K2.5 shape, top-8 Zipf(1.1). A sample of
    tokens against the oracle; every sampled token's row equal, bit for bit, to a batch of one."""
    _say("[mxfp4] c4 Kimi shape: 64 tokens x top-8 over 384 experts")
    from vib3_amd.mxfp4 import zipf_picks
    hidden, inter, E, T, k = 7168, 2048, 384, 64, 8
    bank = _bank(hidden, inter, E)
    ids, w = zipf_picks(T, E, k, s=1.1, seed=SEED)
    x, xh = _x(T, hidden)
    got = _run(bank, x, ids, w)
    sample = [0, 17, 63]
    ref = _oracle(bank, xh, ids, w, tokens=sample)
    _check(got[sample], ref)
    for t in sample:
        one = _run(bank, x[t:t + 1].contiguous(), ids[t:t + 1].copy(), w[t:t + 1].copy())
        _check(one, got[t:t + 1])
    # a second launch may place an expert's entries in another order (the grouping takes
    # places from counting atomics); the output must not change
    again = _run(bank, x, ids, w)
    assert np.array_equal(again, got)


def test_argument_errors():
    from vib3_amd import _lib
    from vib3_amd.mxfp4 import MoeMxfp4Batch
    bank = _bank(256, 256, 4)
    b = MoeMxfp4Batch(bank, 2, 2)
    x, _ = _x(2, 256)
    ids = torch.zeros((2, 2), dtype=torch.int16, device="cuda")
    w = torch.ones((2, 2), dtype=torch.float32, device="cuda")
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    d = b.desc(x, ids, w)
    d.hidden = 200
    assert lib.vib3_launch_moe_mxfp4_batched(d, st) == -1
    d = b.desc(x, ids, w)
    d.workspace_bytes = 16
    assert lib.vib3_launch_moe_mxfp4_batched(d, st) == -4
    d = b.desc(x, ids, w)
    d.tokens = 5000
    assert lib.vib3_launch_moe_mxfp4_batched(d, st) == -2
    d = b.desc(x, ids, w)
    d.ids = None
    assert lib.vib3_launch_moe_mxfp4_batched(d, st) == -3


def test_graph_replay_equals_eager():
    """The batched launch (grouping, then the one-token rows, two-token rows and matrix-core
    chains on three streams, then the combine) captured in a HIP graph: the fork and join
    become graph edges, and three replays with new activations, ids and weights each equal an
    eager launch bit for bit."""
    from vib3_amd.mxfp4 import MoeMxfp4Batch
    _say("case: mxfp4 batch graph capture + replays")
    hidden, inter, E, T, k = 512, 768, 12, 24, 4
    bank = _bank(hidden, inter, E, layer=3)
    rng = np.random.default_rng(9)

    def picks():
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint16)
        ids[: T // 2, 0] = 5  # a hot expert (matrix-core path) beside one- and two-token ones
        ids[: T // 2, 1:] = np.where(ids[: T // 2, 1:] == 5, 6, ids[: T // 2, 1:])
        w = rng.random((T, k)).astype(np.float32)
        return ids, w

    g = MoeMxfp4Batch(bank, T, k)
    ref = MoeMxfp4Batch(bank, T, k)
    xb, _ = _x(T, hidden, 80)
    xb = xb.clone()
    ids0, w0 = picks()
    ib = torch.from_numpy(ids0.view(np.int16)).cuda()
    wb = torch.from_numpy(w0).cuda()
    g.launch(xb, ib, wb)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        g.launch(xb, ib, wb)
    torch.cuda.synchronize()
    for r in range(3):
        xt, _ = _x(T, hidden, 81 + r)
        ids, w = picks()
        xb.copy_(xt)
        ib.copy_(torch.from_numpy(ids.view(np.int16)).cuda())
        wb.copy_(torch.from_numpy(w).cuda())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = g.out.view(torch.int16).cpu().numpy().copy()
        want = ref.launch(xt, torch.from_numpy(ids.view(np.int16)).cuda(),
                          torch.from_numpy(w).cuda())
        torch.cuda.synchronize()
        _say(f"  replay {r}")
        assert np.array_equal(got, want.view(torch.int16).cpu().numpy())
    del graph
