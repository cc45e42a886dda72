"""Batched decode over MXFP4 experts resident in HBM (host side, torch for memory).

T tokens each pick top_k experts; the library groups the picks per expert and runs every touched
expert once for all of its tokens as a grouped GEMM on the matrix cores
(``vib3_launch_moe_mxfp4_batched``). Per token the result is the engine's expert composition
(src/runtime/engine.rs:5801-6306) with MXFP4 weights: E2M1 codes (cuda/src/kernels.cu:438-441)
times E8M0 scales per 32 along k (kernels.cu:2770-2777).

MXFP4 page: [rows x k/2] code bytes (low nibble = even k), then [rows x k/32] E8M0 bytes.
Expert e's pages are listed in a device table u64[E][3] (0 = up, 1 = gate, 2 = down).
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import MoeMxfp4Batch as BatchDesc
from .moe import matrix_stream

SEG_UP, SEG_GATE, SEG_DOWN = 0, 1, 2


def mxfp4_page_bytes(rows: int, k: int) -> int:
    return rows * (k // 2) + rows * (k // 32)


def zipf_picks(tokens: int, num_experts: int, top_k: int, s: float = 1.1, seed: int = 0):
    """Seeded top_k distinct experts per token, Zipf(s)-skewed over a seeded rank permutation,
    with positive weights that sum to 1 per token. Returns (ids u16 [T, k], weights f32 [T, k])."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(num_experts)  # rank r -> expert perm[r]
    p = 1.0 / np.arange(1, num_experts + 1, dtype=np.float64) ** s
    p /= p.sum()
    ids = np.empty((tokens, top_k), dtype=np.uint16)
    for t in range(tokens):
        ranks = rng.choice(num_experts, size=top_k, replace=False, p=p)
        ids[t] = perm[ranks]
    w = rng.random((tokens, top_k)).astype(np.float32) + np.float32(0.05)
    w /= w.sum(axis=1, keepdims=True)
    return ids, w.astype(np.float32)


class Mxfp4ExpertBank:
    """Every expert (up, gate, down) of one layer as MXFP4 pages in one HBM buffer."""

    def __init__(self, hidden: int, inter: int, num_experts: int, layer: int = 0,
                 seed: int = 0x5EED0004, device="cuda"):
        self.hidden, self.inter, self.num_experts = hidden, inter, num_experts
        self.layer, self.seed = layer, seed
        self.device = torch.device(device)
        dims = [(inter, hidden), (inter, hidden), (hidden, inter)]  # (rows, k) per segment
        self.dims = dims
        sizes = [(mxfp4_page_bytes(r, k) + 255) // 256 * 256 for r, k in dims]
        self.expert_bytes = sum(sizes)
        self.nbytes = self.expert_bytes * num_experts
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=self.device)
        base = self.buf.data_ptr()
        table = np.empty((num_experts, 3), dtype=np.uint64)
        st = torch.cuda.current_stream(self.device).cuda_stream
        for e in range(num_experts):
            off = e * self.expert_bytes
            for sgi, (rows, k) in enumerate(dims):
                addr = base + off
                table[e, sgi] = addr
                _lib.call("vib3_synth_mxfp4_page", addr, seed,
                          matrix_stream(layer, e, sgi), k, 0, rows, st)
                off += sizes[sgi]
        self.table_host = table
        self.table = torch.from_numpy(table.view(np.int64)).to(self.device)

    def expert_pages_host(self, e: int):
        """(up, gate, down) pages of expert e, copied back from the device."""
        out = []
        for sgi, (rows, k) in enumerate(self.dims):
            off = int(self.table_host[e, sgi]) - self.buf.data_ptr()
            out.append(self.buf[off:off + mxfp4_page_bytes(rows, k)].cpu().numpy())
        return tuple(out)


class MoeMxfp4Batch:
    """Launcher for one batch shape: owns the workspace for `tokens` x `top_k` picks."""

    def __init__(self, bank: Mxfp4ExpertBank, tokens: int, top_k: int):
        self.bank, self.tokens, self.top_k = bank, tokens, top_k
        d = self._desc(None, None, None, None)
        n = _lib.load().vib3_moe_mxfp4_workspace_bytes(d)
        self.workspace = torch.empty(n + 256, dtype=torch.uint8, device=bank.device)
        self.out = torch.empty((tokens, bank.hidden), dtype=torch.bfloat16, device=bank.device)

    def _desc(self, x, ids, weights, out) -> BatchDesc:
        b = self.bank
        d = BatchDesc()
        d.x = x.data_ptr() if x is not None else None
        d.tokens, d.hidden, d.inter = self.tokens, b.hidden, b.inter
        d.num_experts, d.top_k = b.num_experts, self.top_k
        d.ids = ids.data_ptr() if ids is not None else None
        d.weights = weights.data_ptr() if weights is not None else None
        d.page_table = b.table.data_ptr()
        d.out = out.data_ptr() if out is not None else None
        if hasattr(self, "workspace"):
            base = self.workspace.data_ptr()
            d.workspace = (base + 255) // 256 * 256
            d.workspace_bytes = self.workspace.numel() - (d.workspace - base)
        return d

    def desc(self, x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
             out: Optional[torch.Tensor] = None) -> BatchDesc:
        assert x.dtype == torch.bfloat16 and x.shape == (self.tokens, self.bank.hidden)
        assert ids.dtype == torch.int16 and ids.shape == (self.tokens, self.top_k)
        assert weights.dtype == torch.float32 and weights.shape == (self.tokens, self.top_k)
        return self._desc(x, ids, weights, self.out if out is None else out)

    def launch(self, x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
        d = self.desc(x, ids, weights)
        st = torch.cuda.current_stream(self.bank.device).cuda_stream
        rc = _lib.load().vib3_launch_moe_mxfp4_batched(d, st)
        if rc:
            raise _lib.Vib3Error("vib3_launch_moe_mxfp4_batched", rc)
        return self.out
