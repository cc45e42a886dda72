"""The fused layer run on weights read from a .vib3 file (vib3_amd.vib3file.load_moe_layer):
pages uploaded into a device pool, page tables built from the catalog (several pages per
segment), router / norm / shared gate read from the layer's shared tensors. Checked against
the oracle's composition on the file's own pages: ids bit-exact where the margin exceeds 1e-3,
output rel-L2 <= 1e-3."""
import numpy as np
import pytest

from oracle import oracle as O
from vib3_writer import make_test_model

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("with_shared", [True, False])
def test_layer_from_file(tmp_path, with_shared):
    from vib3_amd.vib3file import Vib3File, load_moe_layer
    print(f"case: layer from a .vib3 file, shared={with_shared}", flush=True)
    path = str(tmp_path / "m.vib3")
    cfg, dense = make_test_model(path, with_shared=with_shared)
    hidden, inter, E, k = 1024, 256, 8, 2
    with Vib3File(path) as f:
        layer = load_moe_layer(f, 0)
        assert layer.bank.rows_per_page == [96, 96, 400]
        assert layer.bank.shape.group_size == 32
        x = O.synth_normal_array(0x5EED0007, 0x9100, 0, hidden, 15.0, O.F32)
        res = O.synth_normal_array(0x5EED0007, 0x9101, 0, hidden, 15.0, O.F32)
        out = layer.launch(torch.from_numpy(x).cuda(),
                           residual=torch.from_numpy(res).cuda()).cpu().numpy()
        torch.cuda.synchronize()
        xn = O.rms_norm_f32(x, dense["norm"], 1e-6)
        r_ids, r_wts, r_scores = O.router(xn, dense["router"], O.F16, E, hidden, k, 1, 2.827,
                                          True, None)
        keys = np.sort(1 / (1 + np.exp(-r_scores.astype(np.float64))))[::-1]
        assert keys[k - 1] - keys[k] > 1e-3, "selection margin below 1e-3: choose another x"
        assert layer.ids.cpu().numpy().view(np.uint16)[:k].tolist() == r_ids.tolist()
        routed = {int(e): layer.bank.expert_pages_host(int(e)) for e in r_ids}
        shared = [layer.bank.expert_pages_host(E)] if with_shared else []
        gates = [O.sigmoid(O.linear_row_f16(xn, dense["gate"]))] if with_shared else None
        ref = O.moe_layer(xn, hidden, inter, 32, O.BF16, routed, r_ids, r_wts, shared,
                          faithful=True, shared_weights=gates)
        ref = O.residual_add_f32(res, ref)
        rel = rel_l2(out, ref)
        print(f"  rel_l2={rel:.3e}", flush=True)
        assert rel <= 1e-3
        assert rel_l2(out - res, ref - res) <= 1e-3
