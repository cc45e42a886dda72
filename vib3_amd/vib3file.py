"""Run the fused MoE layer on weights read from a `.vib3` model file (format.rs).

`Vib3File` wraps the C reader of libvib3_hip (vib3_file_* in include/vib3_hip.h; the file is
memory-mapped, pages come back as host pointers). `load_moe_layer` uploads one layer's expert
pages into a device pool, builds the page tables with `vib3_build_page_table` (the device form
of `plan_layer_resident` / engine.rs:1236-1299, several pages per segment), loads the router
(segment 3), the pre-MoE norm (segment 7) and the shared-expert gate (segment 26) of the layer's
shared tensors (expert 0xFFFF), and returns a `moe.MoeInt4Layer` ready to launch.

Segments (types.rs:200 PageId.segment): routed experts 0 = up, 1 = gate, 2 = down; the
layer's shared tensors (expert 0xFFFF) 3 = router, 7 = MoE norm, 14/15/16 = shared expert
up/gate/down, 26 = shared expert sigmoid gate. INT4 pages are the converter's layout
(convert.rs:1807-1880): [rows x k/2] nibbles then [rows x k/g] 2-byte scales, BF16 as the
reference quantizer writes them (kernels.rs:3804).
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from . import _lib
from .moe import BankShape, MoeInt4Layer

EXPERT_SHARED = 0xFFFF
SEG_UP, SEG_GATE, SEG_DOWN = 0, 1, 2
SEG_ROUTER, SEG_MOE_NORM = 3, 7
SEG_SHARED_UP, SEG_SHARED_GATE, SEG_SHARED_DOWN, SEG_SHARED_SIGMOID = 14, 15, 16, 26
DTYPE_FP16, DTYPE_BF16, DTYPE_INT4 = 0, 1, 5  # types.rs:633


class FileInfo(C.Structure):
    _fields_ = [("num_layers", C.c_uint32), ("num_experts", C.c_uint32),
                ("num_active_experts", C.c_uint32), ("hidden_dim", C.c_uint32),
                ("expert_hidden_dim", C.c_uint32), ("expert_dtype", C.c_uint8),
                ("shared_dtype", C.c_uint8), ("page_count", C.c_uint32),
                ("page_data_offset", C.c_uint64), ("page_data_size", C.c_uint64)]


class PageEntry(C.Structure):
    _fields_ = [("layer", C.c_uint16), ("expert", C.c_uint16), ("segment", C.c_uint16),
                ("page_idx", C.c_uint16), ("file_offset", C.c_uint64),
                ("compressed_size", C.c_uint32), ("raw_size", C.c_uint32),
                ("row_start", C.c_uint16), ("row_count", C.c_uint16), ("col_start", C.c_uint16),
                ("col_count", C.c_uint16), ("compression", C.c_uint8), ("flags", C.c_uint8),
                ("catalog_index", C.c_uint32)]


def _check(name: str, rc: int) -> None:
    if rc != 0:
        raise _lib.Vib3Error(name, rc)


class Vib3File:
    """A `.vib3` file opened through the library's reader (format.rs:241 Vib3File::open)."""

    def __init__(self, path: str) -> None:
        self._lib = _lib.load()
        self._h = C.c_void_p()
        _check("vib3_file_open", self._lib.vib3_file_open(path.encode(), C.byref(self._h)))
        self.info = FileInfo()
        _check("vib3_file_get_info", self._lib.vib3_file_get_info(self._h, C.byref(self.info)))
        js, n = C.c_char_p(), C.c_size_t()
        _check("vib3_file_metadata", self._lib.vib3_file_metadata(self._h, C.byref(js), C.byref(n)))
        self.metadata = json.loads(C.string_at(js, n.value).decode()) if n.value else {}

    def close(self) -> None:
        if self._h:
            self._lib.vib3_file_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def page(self, index: int) -> PageEntry:
        e = PageEntry()
        _check("vib3_file_page", self._lib.vib3_file_page(self._h, index, C.byref(e)))
        return e

    def expert_pages(self, layer: int, expert: int) -> List[PageEntry]:
        """format.rs:371 pages_for_expert."""
        n = C.c_int()
        _check("vib3_file_expert_pages",
               self._lib.vib3_file_expert_pages(self._h, layer, expert, None, 0, C.byref(n)))
        out = (PageEntry * max(n.value, 1))()
        _check("vib3_file_expert_pages",
               self._lib.vib3_file_expert_pages(self._h, layer, expert, out, n.value, C.byref(n)))
        return list(out[: n.value])

    def page_bytes(self, index: int) -> np.ndarray:
        """A page's bytes: a read-only view of the mapping, or the decompressed copy of an LZ4
        page (format.rs:501 read_page_sync)."""
        e = self.page(index)
        if e.compression != 0:
            out = np.empty(e.raw_size, dtype=np.uint8)
            n = C.c_size_t()
            _check("vib3_file_read_page", self._lib.vib3_file_read_page(
                self._h, index, out.ctypes.data, out.size, C.byref(n)))
            return out[: n.value]
        p, n = C.c_void_p(), C.c_size_t()
        _check("vib3_file_page_data",
               self._lib.vib3_file_page_data(self._h, index, C.byref(p), C.byref(n)))
        buf = (C.c_uint8 * n.value).from_address(p.value)
        return np.frombuffer(buf, dtype=np.uint8)

    def segment_bytes(self, layer: int, expert: int, segment: int) -> np.ndarray:
        """A segment's pages concatenated in page order (a dense tensor such as the router)."""
        pages = [e for e in self.expert_pages(layer, expert) if e.segment == segment]
        if not pages:
            raise KeyError(f"layer {layer} expert {expert:#x} has no segment {segment}")
        return np.concatenate([self.page_bytes(e.catalog_index) for e in pages])

    def build_page_table(self, layer: int, experts: List[int], segments, page_addr: np.ndarray,
                         max_pages: int, rows_required=None):
        """vib3_build_page_table: host u64[len(experts)][3][max_pages] and rows per page.
        rows_required (3 ints): rows each segment must cover (None: the file's dimensions)."""
        table = np.zeros(len(experts) * 3 * max_pages, dtype=np.uint64)
        rpp = (C.c_int * 3)()
        ex = np.asarray(experts, dtype=np.uint16)
        seg = np.asarray(segments, dtype=np.uint16)
        pa = np.ascontiguousarray(page_addr, dtype=np.uint64)
        req = (C.c_int * 3)(*rows_required) if rows_required is not None else None
        _check("vib3_build_page_table", self._lib.vib3_build_page_table(
            self._h, layer, ex.ctypes.data, len(experts), seg.ctypes.data, pa.ctypes.data,
            table.ctypes.data, max_pages, rpp, req))
        return table, list(rpp)


@dataclass
class FileExpertBank:
    """The device side of one layer read from a file: what MoeInt4Layer needs from a bank."""
    shape: BankShape
    pool: torch.Tensor            # every uploaded page, 256-byte aligned
    routed_table: torch.Tensor
    shared_table: Optional[torch.Tensor]
    max_pages: int
    rows_per_page: List[int]
    device: torch.device
    file: "Vib3File"
    layer: int

    def expert_pages_host(self, expert: int):
        """Host copies of expert `expert`'s pages (E + s: shared expert s) per segment, and the
        rows per page: the form the CPU oracle takes."""
        E = self.shape.num_experts
        segs = (SEG_UP, SEG_GATE, SEG_DOWN) if expert < E else \
            (SEG_SHARED_UP, SEG_SHARED_GATE, SEG_SHARED_DOWN)
        entries = self.file.expert_pages(self.layer, expert if expert < E else EXPERT_SHARED)
        pages = []
        for s in segs:
            ps = sorted((p for p in entries if p.segment == s), key=lambda p: p.page_idx)
            pages.append([np.array(self.file.page_bytes(p.catalog_index)) for p in ps])
        return pages, list(self.rows_per_page)


def _group_size(entry: PageEntry, k: int) -> int:
    """The scale group of an INT4 page from its size: raw = rows * (k/2 + 2 * ceil(k/g))."""
    per_row = entry.raw_size // max(entry.row_count, 1)
    ng = (per_row - (k + 1) // 2) // 2
    if ng <= 0 or per_row * entry.row_count != entry.raw_size:
        raise ValueError("page size does not match an INT4 row layout")
    g = -(-k // ng)
    if -(-k // g) != ng:
        raise ValueError("no group size gives this page's scale count")
    return g


def load_moe_layer(f: Vib3File, layer: int, device="cuda", scale_dtype: int = _lib.DT_BF16,
                   **layer_kwargs) -> MoeInt4Layer:
    """Upload layer `layer`'s routed and shared INT4 experts and its router / norm / gate
    tensors, and return the fused layer over them (router settings from the file's metadata
    unless given in layer_kwargs)."""
    meta = f.metadata
    info = f.info
    if info.expert_dtype != DTYPE_INT4:
        raise ValueError("load_moe_layer reads INT4 experts (expert_dtype 5)")
    device = torch.device(device)
    hidden, inter, E = int(info.hidden_dim), int(info.expert_hidden_dim), int(info.num_experts)
    routed = [(e, f.expert_pages(layer, e)) for e in range(E)]
    shared_entries = f.expert_pages(layer, EXPERT_SHARED)
    has_shared = any(p.segment == SEG_SHARED_UP for p in shared_entries)

    # one pool holding every expert page of the layer, each page 256-byte aligned
    wanted = [p for _, ps in routed for p in ps if p.segment in (SEG_UP, SEG_GATE, SEG_DOWN)]
    wanted += [p for p in shared_entries
               if p.segment in (SEG_SHARED_UP, SEG_SHARED_GATE, SEG_SHARED_DOWN)]
    offs, total = {}, 0
    for p in wanted:
        offs[p.catalog_index] = total
        total += (p.raw_size + 255) // 256 * 256
    pool = torch.empty(max(total, 256), dtype=torch.uint8, device=device)
    host = np.zeros(pool.numel(), dtype=np.uint8)
    for p in wanted:
        data = f.page_bytes(p.catalog_index)
        host[offs[p.catalog_index]: offs[p.catalog_index] + data.size] = data
    pool.copy_(torch.from_numpy(host))
    base = pool.data_ptr()
    page_addr = np.zeros(info.page_count, dtype=np.uint64)
    for q, o in offs.items():
        page_addr[q] = base + o
    max_pages = max([p.page_idx + 1 for p in wanted] or [1])

    table, rpp = f.build_page_table(layer, list(range(E)), (SEG_UP, SEG_GATE, SEG_DOWN),
                                    page_addr, max_pages)
    shared_table, s_rpp = None, None
    if has_shared:
        shared_table, s_rpp = f.build_page_table(
            layer, [EXPERT_SHARED], (SEG_SHARED_UP, SEG_SHARED_GATE, SEG_SHARED_DOWN),
            page_addr, max_pages)
        if s_rpp != rpp:
            raise ValueError("shared and routed experts must share rows per page")
    up0 = next(p for p in wanted if p.segment == SEG_UP)
    g = _group_size(up0, hidden)

    shape = BankShape(hidden=hidden, inter=inter, group_size=g, scale_dtype=scale_dtype,
                      scale_sigma=0.0, num_experts=E, num_shared=1 if has_shared else 0)
    bank = FileExpertBank(
        shape=shape, pool=pool, routed_table=torch.from_numpy(table.view(np.int64)).to(device),
        shared_table=torch.from_numpy(shared_table.view(np.int64)).to(device)
        if shared_table is not None else None,
        max_pages=max_pages, rows_per_page=rpp, device=device, file=f, layer=layer)

    def shared_tensor(seg, dtype):
        if not any(p.segment == seg for p in shared_entries):
            return None
        raw = f.segment_bytes(layer, EXPERT_SHARED, seg)
        return torch.from_numpy(raw.copy()).to(device).view(dtype)

    wdt = torch.float16 if info.shared_dtype == DTYPE_FP16 else torch.bfloat16
    router_w = shared_tensor(SEG_ROUTER, wdt)
    if router_w is not None:
        router_w = router_w[: E * hidden]
    norm_w = shared_tensor(SEG_MOE_NORM, torch.float16)
    gate_w = shared_tensor(SEG_SHARED_SIGMOID, torch.float16) if has_shared else None
    sigmoid = meta.get("scoring_func", "softmax") == "sigmoid"
    kw = dict(top_k=int(meta.get("num_active_experts", info.num_active_experts)),
              scoring_mode=_lib.ROUTER_SIGMOID if sigmoid else _lib.ROUTER_SOFTMAX,
              scaling_factor=float(meta.get("routed_scaling_factor", 1.0) or 1.0)
              if sigmoid else 1.0,
              normalize=bool(meta.get("norm_topk_prob", True)),
              norm_weight=norm_w[:hidden] if norm_w is not None else None,
              norm_eps=float(meta.get("rms_norm_eps", 1e-6)),
              shared_gate=gate_w[:hidden] if gate_w is not None else None)
    kw.update(layer_kwargs)
    return MoeInt4Layer(bank, router_w, None, **kw)


def build_page_table_resolved(pages, experts: List[int], segments, max_pages: int,
                              rows_required=None):
    """vib3_build_page_table_resolved over planner pages, each (layer, expert, segment,
    page_idx, device_ptr, row_start, row_count). Returns (table u64[len(experts)*3*max_pages],
    rows_per_page, missing): missing lists the indices of non-resident pages (device_ptr 0),
    in which case the table must not be launched."""
    lib = _lib.load()
    arr = (_lib.ResolvedPage * max(len(pages), 1))()
    for i, p in enumerate(pages):
        arr[i] = _lib.ResolvedPage(*p)
    table = np.zeros(len(experts) * 3 * max_pages, dtype=np.uint64)
    rpp = (C.c_int * 3)()
    ex = np.asarray(experts, dtype=np.uint16)
    seg = np.asarray(segments, dtype=np.uint16)
    req = (C.c_int * 3)(*rows_required) if rows_required is not None else None
    missing = np.zeros(max(len(pages), 1), dtype=np.uint32)
    n = C.c_int()
    rc = lib.vib3_build_page_table_resolved(arr, len(pages), ex.ctypes.data, len(experts),
                                            seg.ctypes.data, req, table.ctypes.data, max_pages,
                                            rpp, missing.ctypes.data, missing.size, C.byref(n))
    if rc not in (0, -7):
        raise _lib.Vib3Error("vib3_build_page_table_resolved", rc)
    return table, list(rpp), missing[: n.value].tolist()
