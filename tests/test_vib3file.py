"""The .vib3 reader (vib3_file_*) and the page-table builder on the CPU: header, metadata,
catalog order, page bytes, the table of every expert's segments, and the error paths. The
files come from tests/vib3_writer.py, which follows the reference writer's layout
(format.rs:842-1030). No GPU call."""
import os
import struct

import numpy as np
import pytest

from vib3_writer import make_test_model


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("vib3") / "model.vib3")
    cfg, dense = make_test_model(path)
    return path, cfg, dense


def test_header_metadata_and_catalog(model):
    from vib3_amd.vib3file import Vib3File
    path, cfg, dense = model
    with Vib3File(path) as f:
        i = f.info
        assert (i.num_layers, i.num_experts, i.num_active_experts, i.hidden_dim,
                i.expert_hidden_dim, i.expert_dtype, i.shared_dtype) == (1, 8, 2, 1024, 256, 5, 0)
        assert i.page_count == len(dense["pages"])
        assert i.page_data_offset % (2 << 20) == 0
        assert f.metadata["scoring_func"] == "sigmoid"
        assert f.metadata["routed_scaling_factor"] == pytest.approx(2.827)
        # catalog sorted by (layer, expert, segment, page_idx); expert 3 has 3 + 3 + 3 pages
        e3 = f.expert_pages(0, 3)
        assert [(p.segment, p.page_idx) for p in e3] == [(s, q) for s in range(3) for q in range(3)]
        assert [p.row_start for p in e3[:3]] == [0, 96, 192]
        assert [p.row_count for p in e3[6:]] == [400, 400, 224]
        want = {(p[0], p[1], p[2], p[3]): p[7] for p in dense["pages"]}
        for p in e3 + f.expert_pages(0, 0xFFFF):
            assert f.page_bytes(p.catalog_index).tobytes() == want[(p.layer, p.expert,
                                                                     p.segment, p.page_idx)]
            assert p.file_offset % 4096 == 0
        router = f.segment_bytes(0, 0xFFFF, 3).view(np.uint16)
        assert np.array_equal(router, dense["router"])
        assert f.expert_pages(0, 100) == []


def test_page_table(model):
    from vib3_amd.vib3file import Vib3File
    path, _, _ = model
    with Vib3File(path) as f:
        addr = np.arange(f.info.page_count, dtype=np.uint64) * 4096 + (1 << 40)
        table, rpp = f.build_page_table(0, list(range(8)), (0, 1, 2), addr, 3)
        assert rpp == [96, 96, 400]
        table = table.reshape(8, 3, 3)
        for e in range(8):
            for p in f.expert_pages(0, e):
                assert table[e, p.segment, p.page_idx] == addr[p.catalog_index]
        shared, srpp = f.build_page_table(0, [0xFFFF], (14, 15, 16), addr, 3)
        assert srpp == [96, 96, 400] and np.all(shared != 0)
        # a page that is not resident (address 0) is an error, as is a missing expert
        gap = addr.copy()
        gap[f.expert_pages(0, 5)[1].catalog_index] = 0
        with pytest.raises(Exception) as err:
            f.build_page_table(0, list(range(8)), (0, 1, 2), gap, 3)
        assert getattr(err.value, "code", None) == -7
        # segments must reach the rows the kernels read: the file's 256 / 1024 rows pass,
        # one more row than the pages hold is a truncated segment
        f.build_page_table(0, list(range(8)), (0, 1, 2), addr, 3, rows_required=(256, 256, 1024))
        with pytest.raises(Exception) as err:
            f.build_page_table(0, list(range(8)), (0, 1, 2), addr, 3,
                               rows_required=(256, 257, 1024))
        assert getattr(err.value, "code", None) == -5
        with pytest.raises(Exception):
            f.build_page_table(0, [9], (0, 1, 2), addr, 3)
        with pytest.raises(Exception):  # max_pages too small for the 3 pages of a segment
            f.build_page_table(0, [0], (0, 1, 2), addr, 2)


def test_errors(model, tmp_path):
    from vib3_amd._lib import Vib3Error
    from vib3_amd.vib3file import Vib3File
    path, _, _ = model
    with pytest.raises(Vib3Error) as e:
        Vib3File(str(tmp_path / "missing.vib3"))
    assert e.value.code == -6
    bad = tmp_path / "bad.vib3"
    raw = bytearray(open(path, "rb").read(4096))
    raw[0:8] = struct.pack("<Q", 0x1234)
    bad.write_bytes(bytes(raw))
    with pytest.raises(Vib3Error) as e:
        Vib3File(str(bad))
    assert e.value.code == -5
    trunc = tmp_path / "trunc.vib3"
    trunc.write_bytes(open(path, "rb").read(600))  # the catalog runs past the end
    with pytest.raises(Vib3Error) as e:
        Vib3File(str(trunc))
    assert e.value.code == -5


def test_lz4_pages(tmp_path):
    """LZ4 pages (lz4_flex's size-prepended blocks, format.rs:526) decompress to the raw page;
    zstd pages are refused."""
    from vib3_amd._lib import Vib3Error
    from vib3_amd.vib3file import Vib3File
    from vib3_writer import lz4_compress
    path = str(tmp_path / "lz4.vib3")
    keys = {(0, 1, 2, 0), (0, 1, 0, 1), (0, 0xFFFF, 3, 0)}
    _, dense = make_test_model(path, E=2, compressed=keys, zstd={(0, 0, 1, 0)})
    want = {(p[0], p[1], p[2], p[3]): p[7] for p in dense["pages"]}
    with Vib3File(path) as f:
        seen = 0
        for e in (0, 1, 0xFFFF):
            for p in f.expert_pages(0, e):
                k = (p.layer, p.expert, p.segment, p.page_idx)
                if k == (0, 0, 1, 0):
                    assert p.compression == 2
                    with pytest.raises(Vib3Error) as err:
                        f.page_bytes(p.catalog_index)
                    assert err.value.code == -1
                    continue
                assert p.compression == (1 if k in keys else 0)
                seen += p.compression == 1
                assert f.page_bytes(p.catalog_index).tobytes() == want[k]
        assert seen == 3
    # pages that do compress: long runs (overlapping matches, extended lengths), short
    # repeats, literal runs over 15 bytes, and tiny pages, through the library's decompressor
    rng = np.random.default_rng(3)
    datas = [b"a" * 1000, b"", b"abc", bytes(rng.integers(0, 4, 5000, dtype=np.uint8)),
             bytes(rng.integers(0, 256, 3000, dtype=np.uint8)) * 3,
             b"".join(bytes([i % 7]) * (i % 40 + 1) for i in range(400))]
    from vib3_writer import write_vib3
    cfg = {"num_layers": 1, "num_experts": 1, "num_active_experts": 1, "hidden_dim": 64,
           "expert_hidden_dim": 64, "_expert_dtype_code": 5, "_shared_dtype_code": 0}
    pages = [(0, 0, 0, i, 0, 1, 1, d) for i, d in enumerate(datas)]
    path2 = str(tmp_path / "runs.vib3")
    write_vib3(path2, cfg, pages, compressed={(0, 0, 0, i) for i in range(len(datas))})
    with Vib3File(path2) as f:
        for p in f.expert_pages(0, 0):
            assert p.compression == 1
            assert f.page_bytes(p.catalog_index).tobytes() == datas[p.page_idx]
        ratio = f.expert_pages(0, 0)[0].compressed_size / 1000
        assert ratio < 0.05


def _plan(E, rows, rpp, layer=2, base=1 << 40, skip=()):
    """Planner pages of E experts: segment s of `rows[s]` rows cut into rpp[s]-row pages, in a
    shuffled order; (expert, segment, page) in `skip` are not resident (device_ptr 0)."""
    pages = []
    for e in range(E):
        for s in range(3):
            n = -(-rows[s] // rpp[s])
            for p in range(n):
                r = min(rpp[s], rows[s] - p * rpp[s])
                ptr = 0 if (e, s, p) in skip else base + ((e * 3 + s) * 64 + p) * 4096
                pages.append((layer, e, s, p, ptr, p * rpp[s], r))
    rng = np.random.default_rng(5)
    return [pages[i] for i in rng.permutation(len(pages))]


def test_page_table_from_resolved_pages():
    """query_planner.rs:38-43 ResolvedPage lists (the converter's 520 / 1820-row Kimi pages,
    convert.rs:1853-1865) into the fused layer's table: every (expert, segment, page) lands at
    its address whatever the plan's order; a subset of experts selects their rows."""
    from vib3_amd.vib3file import build_page_table_resolved
    rows, rpp = (2048, 2048, 7168), (520, 520, 1820)
    pages = _plan(6, rows, rpp)
    table, got_rpp, missing = build_page_table_resolved(pages, [4, 1], (0, 1, 2), 4, rows)
    assert got_rpp == list(rpp) and missing == []
    t = table.reshape(2, 3, 4)
    for (layer, e, s, p, ptr, r0, rc) in pages:
        if e in (4, 1):
            assert t[[4, 1].index(e), s, p] == ptr
    assert np.count_nonzero(t) == 2 * (4 + 4 + 4)


def test_page_table_resolved_errors_and_missing():
    from vib3_amd._lib import Vib3Error
    from vib3_amd.vib3file import build_page_table_resolved
    rows, rpp = (2048, 2048, 7168), (520, 520, 1820)
    # non-resident pages: listed (plan indices, in table order), entries left 0
    skip = {(1, 0, 2), (3, 2, 0)}
    pages = _plan(4, rows, rpp, skip=skip)
    table, _, missing = build_page_table_resolved(pages, [0, 1, 2, 3], (0, 1, 2), 4, rows)
    assert [(pages[i][1], pages[i][2], pages[i][3]) for i in missing] == sorted(skip)
    t = table.reshape(4, 3, 4)
    assert t[1, 0, 2] == 0 and t[3, 2, 0] == 0 and t[1, 0, 1] != 0
    # truncated segment: the last down page dropped
    pages = [p for p in _plan(2, rows, rpp) if not (p[2] == 2 and p[3] == 3)]
    with pytest.raises(Vib3Error) as e:
        build_page_table_resolved(pages, [0, 1], (0, 1, 2), 4, rows)
    assert e.value.code == -5
    # a gap (page 1 of up missing) and a short page that is not the last
    pages = [p for p in _plan(1, rows, rpp) if not (p[2] == 0 and p[3] == 1)]
    with pytest.raises(Vib3Error):
        build_page_table_resolved(pages, [0], (0, 1, 2), 4, rows)
    pages = _plan(1, rows, rpp)
    pages = [(a, b, c, d, ptr, r0, 100 if (c == 1 and d == 0) else rc)
             for (a, b, c, d, ptr, r0, rc) in pages]
    with pytest.raises(Vib3Error):
        build_page_table_resolved(pages, [0], (0, 1, 2), 4, rows)
    # an expert absent from the plan, too few table columns, two layers in one plan
    with pytest.raises(Vib3Error):
        build_page_table_resolved(_plan(2, rows, rpp), [0, 5], (0, 1, 2), 4, rows)
    with pytest.raises(Vib3Error) as e:
        build_page_table_resolved(_plan(2, rows, rpp), [0], (0, 1, 2), 3, rows)
    assert e.value.code == -2
    mixed = _plan(1, rows, rpp) + [(3, 0, 0, 9, 1, 0, 1)]
    with pytest.raises(Vib3Error):
        build_page_table_resolved(mixed, [0], (0, 1, 2), 4, rows)
