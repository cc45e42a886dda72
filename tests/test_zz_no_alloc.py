"""vib3_launch_moe_int4_layer_noalloc (the layer with its scratch in a library-held device
array, no caller workspace, no allocation) against vib3_launch_moe_int4_layer on the same
inputs, through the C ABI: identical outputs and ids, on consecutive calls of different shapes
(the Kimi-K2.5 c2 layer, then a smaller layer, then c2 again), and the size limit refused
before any launch."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 0x5EED0002


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _run_both(lib, layer, x):
    """(out, ids) of the workspace entry point, then of the no-allocation one."""
    st = torch.cuda.current_stream().cuda_stream
    d = layer._desc(x)
    assert lib.vib3_launch_moe_int4_layer(d, st) == 0
    torch.cuda.synchronize()
    ref = (layer.out.cpu().numpy().copy(), layer.ids.cpu().numpy().copy())
    layer.out.fill_(float("nan"))
    layer.ids.fill_(-1)
    d = layer._desc(x)
    d.workspace, d.workspace_bytes = None, 0
    assert lib.vib3_launch_moe_int4_layer_noalloc(d, st) == 0
    torch.cuda.synchronize()
    got = (layer.out.cpu().numpy().copy(), layer.ids.cpu().numpy().copy())
    return ref, got


def test_noalloc_matches_workspace_entry_point():
    from vib3_amd import _lib, moe
    from vib3_amd._lib import DT_BF16, ROUTER_SIGMOID, ROUTER_SOFTMAX
    lib = _lib.load()
    _say("case: noalloc c2 Kimi layer, call 1")
    kimi = moe.BankShape(hidden=7168, inter=2048, group_size=32, scale_dtype=DT_BF16,
                         scale_sigma=0.01, num_experts=384, num_shared=1)
    bank = moe.Int4ExpertBank(kimi, layer=0, seed=SEED)
    w, b = moe.make_router(kimi, 0, SEED, 0.01, 0.1)
    big = moe.MoeInt4Layer(bank, w, b, top_k=8, scoring_mode=ROUTER_SIGMOID,
                           scaling_factor=2.827, normalize=True)
    ref, got = _run_both(lib, big, moe.make_activation(kimi.hidden, 0, SEED))
    assert np.array_equal(ref[1], got[1]) and np.array_equal(ref[0], got[0])

    _say("case: noalloc smaller layer, call 2")
    small = moe.BankShape(hidden=1024, inter=256, group_size=32, scale_dtype=DT_BF16,
                          scale_sigma=0.03, num_experts=40, num_shared=1)
    sbank = moe.Int4ExpertBank(small, layer=3, seed=SEED)
    sw, _ = moe.make_router(small, 3, SEED, 0.05, None)
    lsmall = moe.MoeInt4Layer(sbank, sw, None, top_k=6, scoring_mode=ROUTER_SOFTMAX)
    ref, got = _run_both(lib, lsmall, moe.make_activation(small.hidden, 4, SEED))
    assert np.array_equal(ref[1], got[1]) and np.array_equal(ref[0], got[0])

    _say("case: noalloc c2 again after the smaller shape, call 3")
    ref, got = _run_both(lib, big, moe.make_activation(kimi.hidden, 1, SEED))
    assert np.array_equal(ref[1], got[1]) and np.array_equal(ref[0], got[0])

    d = big._desc(None)
    d.workspace, d.workspace_bytes = None, 0
    assert lib.vib3_moe_int4_layer_status(d, 0, torch.cuda.current_stream().cuda_stream) == 0


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """16 slots x 16384 f16 intermediates need 512 KiB: refused with VIB3_ERR_WORKSPACE before
    anything is launched (the pointers are never dereferenced)."""
    from vib3_amd import _lib
    lib = _lib.load()
    _say("case: noalloc size limit")
    d = _lib.MoeInt4Layer()
    d.x = d.out = d.router_w = d.page_table = d.shared_page_table = 0x10000
    d.x_dtype, d.router_w_dtype, d.scale_dtype = 2, 0, 2
    d.hidden, d.inter, d.group_size = 1024, 16384, 32
    d.num_experts, d.top_k, d.num_shared, d.scoring_mode = 40, 15, 1, 0
    d.max_pages = 1
    d.rows_per_page[0], d.rows_per_page[1], d.rows_per_page[2] = 16384, 16384, 1024
    assert lib.vib3_launch_moe_int4_layer_noalloc(C.byref(d), None) == -4
