"""MoE sublayer over page-indexed INT4 experts resident in HBM (host side, torch for memory).

Mirrors the MoE block of vib3's engine (src/runtime/engine.rs:5052-5307): router ->
expert ids/weights on the device -> page-table lookup -> fused gate/up + SwiGLU -> down with the
weighted sum. The page table is the device form of the planner's ResolvedPage lists
(src/runtime/query_planner.rs:38-43): for (expert, segment, page) the page's device address,
segment 0 = up, 1 = gate, 2 = down (src/core/types.rs:200); page p covers rows
[p * rows_per_page, ...) like ResolvedPage.row_start / row_count.

Weights are generated on the device by the library's counter-based generator, so any expert can
be regenerated on the host by the oracle (tests) or copied back (``expert_pages_host``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import DT_BF16, DT_F16, DT_F32
from ._lib import MoeInt4Layer as LayerDesc

SEG_UP, SEG_GATE, SEG_DOWN = 0, 1, 2


def matrix_stream(layer: int, expert: int, seg: int) -> int:
    """Generator stream id of one logical expert matrix (shared experts use ids >= E)."""
    return ((layer * 8192 + expert) * 4 + seg)


def page_bytes(rows: int, k: int, g: int) -> int:
    return rows * ((k + 1) // 2) + rows * ((k + g - 1) // g) * 2


@dataclass
class BankShape:
    hidden: int
    inter: int
    group_size: int = 32
    scale_dtype: int = DT_BF16
    scale_sigma: float = 0.01
    num_experts: int = 384
    num_shared: int = 1

    def seg_dims(self, seg: int):
        """(rows, k) of a segment's matrix."""
        return (self.hidden, self.inter) if seg == SEG_DOWN else (self.inter, self.hidden)

    def expert_bytes(self) -> int:
        return sum(page_bytes(*self.seg_dims(s), self.group_size) for s in range(3))


class Int4ExpertBank:
    """Every expert of one MoE layer in HBM with its device page tables.

    layout="contiguous": each matrix is one page holding all its rows (rows_per_page = rows).
    layout="paged": each matrix is cut into `tile_rows`-row pages placed at shuffled, seeded
    offsets of a `pool_bytes` pool; only the table knows where they are.
    """

    def __init__(self, shape: BankShape, layer: int = 0, seed: int = 0x5EED0002,
                 layout: str = "contiguous", tile_rows: int = 64,
                 pool_bytes: Optional[int] = None, device="cuda", generate: bool = True):
        self.shape, self.layer, self.seed, self.layout = shape, layer, seed, layout
        self.device = torch.device(device)
        n_all = shape.num_experts + shape.num_shared
        if layout == "contiguous":
            self.rows_per_page = [shape.seg_dims(s)[0] for s in range(3)]
        elif layout == "paged":  # tile_rows: one row count for all segments, or three
            self.rows_per_page = list(tile_rows) if isinstance(tile_rows, (tuple, list)) \
                else [tile_rows] * 3
        else:
            raise ValueError(layout)
        self.pages_per_seg = [math.ceil(shape.seg_dims(s)[0] / self.rows_per_page[s])
                              for s in range(3)]
        self.max_pages = max(self.pages_per_seg)
        # (expert, seg, page) -> (byte offset, rows)
        tiles = []
        for e in range(n_all):
            for s in range(3):
                rows, k = shape.seg_dims(s)
                for p in range(self.pages_per_seg[s]):
                    r = min(self.rows_per_page[s], rows - p * self.rows_per_page[s])
                    tiles.append((e, s, p, r, page_bytes(r, k, shape.group_size)))
        # every page starts 256-byte aligned so its rows keep 16-byte alignment
        sizes = np.array([(t[4] + 255) // 256 * 256 for t in tiles], dtype=np.int64)
        if layout == "contiguous":
            offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]])
            total = int(sizes.sum())
        else:
            unit = int(np.gcd.reduce(sizes))
            units = sizes // unit
            pool_units = (pool_bytes or int(sizes.sum())) // unit
            free = pool_units - int(units.sum())
            if free < 0:
                raise ValueError("pool too small for the tiles")
            rng = np.random.default_rng(seed ^ (layer * 0x9E3779B1))
            order = rng.permutation(len(tiles))
            gaps = rng.multinomial(free, np.full(len(tiles) + 1, 1.0 / (len(tiles) + 1)))
            slot_units = np.cumsum(gaps[:-1] + np.concatenate([[0], units[order][:-1]]))
            offsets = np.empty(len(tiles), dtype=np.int64)
            offsets[order] = slot_units * unit
            total = int(pool_units * unit)
        self.pool = torch.empty(total, dtype=torch.uint8, device=self.device)
        base = self.pool.data_ptr()
        table = np.zeros((n_all, 3, self.max_pages), dtype=np.int64)
        self.tiles = []
        for (e, s, p, r, nbytes), off in zip(tiles, offsets):
            table[e, s, p] = base + int(off)
            self.tiles.append((e, s, p, r, int(off)))
        self.table = torch.from_numpy(table).to(self.device)
        self.routed_table = self.table[: shape.num_experts]
        self.shared_table = self.table[shape.num_experts:]
        if generate:
            self.generate()

    def generate(self) -> None:
        sh = self.shape
        st = torch.cuda.current_stream(self.device).cuda_stream
        for e, s, p, r, off in self.tiles:
            rows, k = sh.seg_dims(s)
            _lib.call("vib3_synth_int4_page", self.pool.data_ptr() + off, self.seed,
                      matrix_stream(self.layer, e, s), k, sh.group_size, sh.scale_dtype,
                      sh.scale_sigma, p * self.rows_per_page[s], r, st)

    def expert_pages_host(self, expert: int):
        """Host copies of an expert's pages: ([up pages], [gate pages], [down pages]), rpp."""
        out = []
        for s in range(3):
            segp = []
            for (e, ss, p, r, off) in self.tiles:
                if e == expert and ss == s:
                    n = page_bytes(r, self.shape.seg_dims(s)[1], self.shape.group_size)
                    segp.append(self.pool[off: off + n].cpu().numpy())
            out.append(segp)
        return out, list(self.rows_per_page)

    def resolved_pages(self, experts: Optional[Sequence[int]] = None):
        """The bank as the query planner's ResolvedPage list (query_planner.rs:38-43): one
        (layer, expert, segment, page_idx, device_ptr, row_start, row_count) per page of the
        given experts (default: every routed expert); shared expert s is expert 0xFFFF with
        segments 14/15/16 (types.rs:203)."""
        E = self.shape.num_experts
        want = set(range(E) if experts is None else experts)
        base = self.pool.data_ptr()
        out = []
        for e, s, p, r, off in self.tiles:
            if e < E and e in want:
                out.append((self.layer, e, s, p, base + off, p * self.rows_per_page[s], r))
            elif e >= E and e in want:
                out.append((self.layer, 0xFFFF, 14 + s, p, base + off,
                            p * self.rows_per_page[s], r))
        return out

    @property
    def nbytes(self) -> int:
        return self.pool.numel()


class MoeInt4Layer:
    """One MoE sublayer: router weights + expert bank + workspace; launch() runs it."""

    def __init__(self, bank: Int4ExpertBank, router_w: Optional[torch.Tensor],
                 router_bias: Optional[torch.Tensor], top_k: int, scoring_mode: int,
                 scaling_factor: float = 1.0, normalize: bool = True, flags: int = 0,
                 norm_weight: Optional[torch.Tensor] = None, norm_eps: float = 1e-6,
                 shared_gate: Optional[torch.Tensor] = None):
        """norm_weight (f16 [hidden]): launch() takes the f32 residual stream and normalises it
        inside the layer; shared_gate (f16 [num_shared][hidden]): sigmoid-gated shared
        experts. launch(..., residual=r) returns r + sublayer."""
        self.bank, self.router_w, self.router_bias = bank, router_w, router_bias
        self.norm_weight, self.norm_eps, self.shared_gate = norm_weight, norm_eps, shared_gate
        self.top_k, self.scoring_mode = top_k, scoring_mode
        self.scaling_factor, self.normalize, self.flags = scaling_factor, normalize, flags
        dev = bank.device
        self.out = torch.empty(bank.shape.hidden, dtype=torch.float32, device=dev)
        self.ids = torch.empty(max(top_k, 1), dtype=torch.int16, device=dev)
        self.wts = torch.empty(max(top_k, 1), dtype=torch.float32, device=dev)
        self.scores = torch.empty(bank.shape.num_experts, dtype=torch.float32, device=dev)
        desc = self._desc(None)
        nbytes = _lib.load().vib3_moe_int4_workspace_bytes(desc)
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def _desc(self, x: Optional[torch.Tensor], in_ids=None, in_wts=None) -> LayerDesc:
        b, sh = self.bank, self.bank.shape
        d = LayerDesc()
        if x is not None:
            d.x = x.data_ptr()
            d.x_dtype = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}[x.dtype]
        d.hidden, d.inter, d.group_size, d.scale_dtype = sh.hidden, sh.inter, sh.group_size, sh.scale_dtype
        if self.router_w is not None:
            d.router_w = self.router_w.data_ptr()
            d.router_w_dtype = {torch.float32: DT_F32, torch.float16: DT_F16,
                                torch.bfloat16: DT_BF16}[self.router_w.dtype]
        d.router_bias = self.router_bias.data_ptr() if self.router_bias is not None else None
        d.num_experts, d.top_k = sh.num_experts, self.top_k
        d.scoring_mode, d.scaling_factor, d.normalize = self.scoring_mode, self.scaling_factor, int(self.normalize)
        d.in_ids = in_ids.data_ptr() if in_ids is not None else None
        d.in_weights = in_wts.data_ptr() if in_wts is not None else None
        d.page_table = b.routed_table.data_ptr()
        d.shared_page_table = b.shared_table.data_ptr() if sh.num_shared else None
        d.num_shared = sh.num_shared
        d.max_pages = b.max_pages
        for s in range(3):
            d.rows_per_page[s] = b.rows_per_page[s]
        d.flags = self.flags
        d.out = self.out.data_ptr()
        d.out_ids = self.ids.data_ptr()
        d.out_weights = self.wts.data_ptr()
        d.out_scores = self.scores.data_ptr()
        if self.norm_weight is not None:
            d.norm_weight = self.norm_weight.data_ptr()
            d.norm_eps = self.norm_eps
        if self.shared_gate is not None:
            d.shared_gate = self.shared_gate.data_ptr()
        if hasattr(self, "workspace"):
            d.workspace = self.workspace.data_ptr()
            d.workspace_bytes = self.workspace.numel()
        return d

    def launch(self, x: torch.Tensor, in_ids: Optional[torch.Tensor] = None,
               in_wts: Optional[torch.Tensor] = None, stream=None,
               residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        if not x.is_cuda or not x.is_contiguous():
            raise TypeError("x must be a contiguous device tensor")
        desc = self._desc(x, in_ids, in_wts)
        if residual is not None:
            if residual.dtype != torch.float32 or residual.numel() != self.bank.shape.hidden:
                raise TypeError("residual must be f32 [hidden]")
            desc.residual = residual.data_ptr()
        st = (stream or torch.cuda.current_stream(x.device)).cuda_stream
        rc = _lib.load().vib3_launch_moe_int4_layer(desc, st)
        if rc != 0:
            raise _lib.Vib3Error("vib3_launch_moe_int4_layer", rc)
        return self.out

    def status(self, clear: bool = False, stream=None) -> int:
        """1 when a launch's router wait gave up since the last clear, else 0 (synchronises)."""
        st = (stream or torch.cuda.current_stream(self.bank.device)).cuda_stream
        rc = _lib.load().vib3_moe_int4_layer_status(self._desc(None), int(clear), st)
        if rc < 0:
            raise _lib.Vib3Error("vib3_moe_int4_layer_status", rc)
        return rc


def make_router(shape: BankShape, layer: int, seed: int, sigma: float, bias_sigma: Optional[float],
                dtype=torch.float32, device="cuda"):
    """Synthetic router weight [E, hidden] ~ N(0, sigma) and bias [E] ~ N(0, bias_sigma)."""
    dt = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}[dtype]
    w = torch.empty(shape.num_experts, shape.hidden, dtype=dtype, device=device)
    st = torch.cuda.current_stream(w.device).cuda_stream
    _lib.call("vib3_synth_normal", w.data_ptr(), dt, w.numel(), seed, 0xF0000000 + layer, 0,
              sigma, st)
    b = None
    if bias_sigma is not None:
        b = torch.empty(shape.num_experts, dtype=torch.float32, device=device)
        _lib.call("vib3_synth_normal", b.data_ptr(), DT_F32, b.numel(), seed, 0xF1000000 + layer,
                  0, bias_sigma, st)
    return w, b


def make_activation(n: int, token: int, seed: int, dtype=torch.bfloat16, device="cuda"):
    """Synthetic activation x[n] ~ N(0, 1) for token index `token`."""
    dt = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}[dtype]
    x = torch.empty(n, dtype=dtype, device=device)
    _lib.call("vib3_synth_normal", x.data_ptr(), dt, n, seed, 0xF2000000 + token, 0, 1.0,
              torch.cuda.current_stream(x.device).cuda_stream)
    return x
