"""Writes small `.vib3` files for the reader's tests, in the layout of the reference writer
(format.rs:842-1030 Vib3Writer::finalize): 512-byte header, JSON metadata, page catalog
sorted by (layer, expert, segment, page_idx), expert index, no vector index / coactivation /
views, page data starting at a 2 MiB boundary with every page 4 KiB aligned. Test helper only.
"""
from __future__ import annotations

import json
import struct

import numpy as np

MAGIC = 0x3342495600000001
PAGE_SIZE = 2 * 1024 * 1024


def lz4_compress(data: bytes) -> bytes:
    """A greedy LZ4 block compressor (4-byte hash matches) in lz4_flex's size-prepended form:
    little-endian raw size, then sequences; the last 5 bytes are literals and no match starts
    in the last 12 (the LZ4 block format's end rules)."""
    data = bytes(data)
    n = len(data)
    out = bytearray(struct.pack("<I", n))
    table = {}
    i = anchor = 0
    limit = n - 12

    def length_bytes(v):
        b = bytearray()
        while v >= 255:
            b.append(255)
            v -= 255
        b.append(v)
        return b

    def emit(lit, mlen, off):
        tok_l = min(len(lit), 15)
        tok_m = 0 if mlen is None else min(mlen - 4, 15)
        out.append((tok_l << 4) | tok_m)
        if tok_l == 15:
            out.extend(length_bytes(len(lit) - 15))
        out.extend(lit)
        if mlen is not None:
            out.extend(struct.pack("<H", off))
            if tok_m == 15:
                out.extend(length_bytes(mlen - 4 - 15))

    while i < limit:
        key = data[i:i + 4]
        cand = table.get(key)
        table[key] = i
        if cand is not None and i - cand <= 0xFFFF:
            m = 4
            while i + m < n - 5 and data[cand + m] == data[i + m]:
                m += 1
            emit(data[anchor:i], m, i - cand)
            i += m
            anchor = i
        else:
            i += 1
    emit(data[anchor:], None, 0)
    return bytes(out)


def write_vib3(path, config: dict, pages, compressed=(), zstd=()):
    """pages: iterable of (layer, expert, segment, page_idx, row_start, row_count, col_count,
    data bytes). Pages whose (layer, expert, segment, page_idx) is in `compressed` are stored
    LZ4-compressed (compression 1); those in `zstd` are only flagged 2 (for the reader's
    refusal path)."""
    meta = json.dumps(config, indent=2).encode()
    stored = []
    for p in pages:
        key = (p[0], p[1], p[2], p[3])
        if key in compressed:
            stored.append((*p[:7], lz4_compress(p[7]), 1, len(p[7])))
        else:
            stored.append((*p, 2 if key in zstd else 0, len(p[7])))
    pages = sorted(stored, key=lambda p: (p[0], p[1], p[2], p[3]))
    cat_off = 512 + len(meta)
    cat_size = 48 * len(pages)
    experts = {}
    for i, p in enumerate(pages):
        experts.setdefault((p[0], p[1]), []).append(i)
    ei_off = cat_off + cat_size
    ei_size = 20 * len(experts)
    end = ei_off + ei_size
    data_off = -(-end // PAGE_SIZE) * PAGE_SIZE
    offs, cur = [], data_off
    for p in pages:
        offs.append(cur)
        cur += -(-len(p[7]) // 4096) * 4096
    header = struct.pack("<QII", MAGIC, 1, 0)
    header += struct.pack("<QQ", 512, len(meta))
    header += struct.pack("<QQI", cat_off, cat_size, len(pages))
    header += struct.pack("<QQ", ei_off, ei_size)
    header += struct.pack("<QQ", end, 0)          # vector index (empty)
    header += struct.pack("<QQ", end, 0)          # coactivation (empty)
    header += struct.pack("<QQI", end, 0, 0)      # views (none)
    header += struct.pack("<QQ", data_off, cur - data_off)
    header += struct.pack("<IIIII", config["num_layers"], config["num_experts"],
                          config["num_active_experts"], config["hidden_dim"],
                          config["expert_hidden_dim"])
    header += struct.pack("<BB", config["_expert_dtype_code"], config["_shared_dtype_code"])
    assert len(header) == 158
    header += bytes(354)
    catalog = b""
    for p, off in zip(pages, offs):
        layer, expert, seg, idx, r0, rc, cc, data, comp, raw = p
        catalog += struct.pack("<HHHHQIIHHHHffHBB4x", layer, expert, seg, idx, off, len(data),
                               raw, r0, rc, 0, cc, 0.0, 0.0, 0, comp, 0)
    index = b""
    for (layer, expert), idx in sorted(experts.items()):
        index += struct.pack("<HHIIIHH", layer, expert, idx[0], len(idx),
                             sum(pages[i][9] for i in idx),
                             len({pages[i][2] for i in idx}), 0)
    with open(path, "wb") as f:
        f.write(header + meta + catalog + index)
        for p, off in zip(pages, offs):
            f.seek(off)
            f.write(bytes(p[7]))
        f.truncate(cur)
    return [o for o in offs]


def int4_pages(layer, expert, segment, full_page: np.ndarray, rows, k, g, rows_per_page):
    """Split one INT4 matrix ([rows x k/2] nibbles + [rows x k/g] scales) into converter-style
    pages of `rows_per_page` rows (convert.rs:1838-1880)."""
    pk, ng = (k + 1) // 2, -(-k // g)
    data = full_page[: rows * pk].reshape(rows, pk)
    sc = full_page[rows * pk:].reshape(rows, ng * 2)
    out = []
    for i, r0 in enumerate(range(0, rows, rows_per_page)):
        r1 = min(rows, r0 + rows_per_page)
        out.append((layer, expert, segment, i, r0, r1 - r0, k,
                    np.concatenate([data[r0:r1].ravel(), sc[r0:r1].ravel()]).tobytes()))
    return out


def dense_pages(layer, expert, segment, raw: bytes, row_bytes, rows_per_page):
    """A dense tensor (router, norm, gate) cut into pages of whole rows."""
    rows = len(raw) // row_bytes
    out = []
    for i, r0 in enumerate(range(0, rows, rows_per_page)):
        r1 = min(rows, r0 + rows_per_page)
        out.append((layer, expert, segment, i, r0, r1 - r0, row_bytes // 2,
                    raw[r0 * row_bytes: r1 * row_bytes]))
    return out


def make_test_model(path, seed=0x5EED0007, hidden=1024, inter=256, E=8, top_k=2,
                    gu_rows_per_page=96, down_rows_per_page=400, router_rows_per_page=3,
                    with_shared=True, compressed=(), zstd=()):
    """A one-layer INT4 MoE model file (Kimi-style: sigmoid router with scaling, one shared
    expert with a sigmoid gate, pre-MoE norm) from the oracle's seeded generator. Returns the
    config and the dense tensors (router / norm / gate f16 bits) for the checks."""
    from oracle import oracle as O
    g = 32
    cfg = {"name": "vib3-test", "architecture": "kimi", "hidden_dim": hidden,
           "expert_hidden_dim": inter, "num_layers": 1, "num_moe_layers": 1,
           "dense_layer_idx": 0, "num_experts": E, "num_active_experts": top_k,
           "num_heads": 8, "num_kv_heads": 8, "max_seq_len": 4096, "vocab_size": 1000,
           "expert_dtype": "INT4", "shared_dtype": "FP16", "rope_theta": 10000.0,
           "rms_norm_eps": 1e-6, "scoring_func": "sigmoid", "routed_scaling_factor": 2.827,
           "norm_topk_prob": True, "num_shared_experts": 1 if with_shared else 0,
           "_expert_dtype_code": 5, "_shared_dtype_code": 0}
    pages = []
    dims = {0: (inter, hidden, gu_rows_per_page), 1: (inter, hidden, gu_rows_per_page),
            2: (hidden, inter, down_rows_per_page)}
    n_all = E + (1 if with_shared else 0)
    for e in range(n_all):
        for s in range(3):
            rows, k, rpp = dims[s]
            full = O.synth_int4_page(seed, 0x100 * e + s, k, g, O.BF16, 0.03, 0, rows)
            if e < E:
                pages += int4_pages(0, e, s, full, rows, k, g, rpp)
            else:
                pages += int4_pages(0, 0xFFFF, 14 + s, full, rows, k, g, rpp)
    router = O.synth_normal_array(seed, 0x9000, 0, E * hidden, 0.05, O.F16)
    norm = (O.synth_normal_array(seed, 0x9001, 0, hidden, 0.1, O.F32) + 1.0).astype(
        np.float16).view(np.uint16)
    gate = O.synth_normal_array(seed, 0x9002, 0, hidden, 0.02, O.F16)
    pages += dense_pages(0, 0xFFFF, 3, router.tobytes(), hidden * 2, router_rows_per_page)
    pages += dense_pages(0, 0xFFFF, 7, norm.tobytes(), hidden * 2, 1)
    if with_shared:
        pages += dense_pages(0, 0xFFFF, 26, gate.tobytes(), hidden * 2, 1)
    write_vib3(path, cfg, pages, compressed=compressed, zstd=zstd)
    return cfg, {"router": router, "norm": norm, "gate": gate, "pages": pages}
