"""MI355X (gfx950) DiT attention hot path: QK-RMSNorm+RoPE and flash attention.

Host-side mirror of the reference's ``diffusers_tpu.kernels`` entry points
over a C-ABI library of hand-written HIP kernels (``include/dt_attention.h``).
"""
from . import _lib
from .kernels import splash
from .kernels.qk_norm_rope import RopeSpec, RopeTable, qk_norm_rope

attention = splash.attention
residual_attention = splash.residual_attention

__all__ = ["attention", "residual_attention", "qk_norm_rope", "RopeSpec",
           "RopeTable",
           "splash", "_lib"]
