"""vib3_amd — MI355X (gfx950) MoE expert compute for vib3: router top-k, INT4 GEMV over
page-indexed expert tiles with fused SwiGLU, behind vib3's C launcher ABI (libvib3_hip.so)."""
from ._lib import DT_BF16, DT_F16, DT_F32, ROUTER_SIGMOID, ROUTER_SOFTMAX, Vib3Error, load

__all__ = ["DT_F32", "DT_F16", "DT_BF16", "ROUTER_SOFTMAX", "ROUTER_SIGMOID", "Vib3Error", "load"]
