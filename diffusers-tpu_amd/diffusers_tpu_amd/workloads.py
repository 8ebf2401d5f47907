"""The BASELINE workloads of the attention path, as seeded synthetic inputs.

Each workload is one attention layer's q/k/v at a DiT shape: pre-norm q, k
``(B, S, H, D)`` and v ``(B, H, S, D)`` ~ N(0, 1) (seeds 0, 1, 2), RMSNorm
weights ~ N(1, 0.02) (seed 3), optional per-head q factor ~ U(0.5, 1.5)
(seed 4), token positions for the RoPE axes, and the padding pattern
(``kv_len``: keys/queries at or past it are padding, zeroed by the prologue
and masked in attention, as models/minimax_h3/jax_dit.py:367-381 and
kernels/splash.py:216-218 do).

Token order: image/video rows first, then text rows (image workloads); the
480p video workload puts its 512 text rows first.  Text rows take position
(0, 0, 0), i.e. the identity rotation (jax_dit.py:727-731).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import torch


@dataclasses.dataclass(frozen=True)
class Workload:
  name: str
  B: int
  H: int
  D: int
  grid: tuple            # (T, Hh, Ww) latent grid of image/video tokens
  text: int = 0          # text rows (appended, or prepended if text_first)
  text_real: int = 0     # real text rows; the rest are padding
  text_first: bool = False
  axis_dims: tuple = (0, 0, 0)
  theta: float = 10000.0
  mode: str = "half"
  eps: float = 1e-6
  head_scale: bool = False
  in_dtype: torch.dtype = torch.bfloat16
  desc: str = ""         # what the BASELINE config is

  @property
  def n_vis(self) -> int:
    return int(np.prod(self.grid))

  @property
  def S(self) -> int:
    return self.n_vis + self.text

  @property
  def kv_len(self) -> int:
    """Real tokens (keys at or past it are padding)."""
    if self.text_first:
      if self.text_real != self.text:
        raise ValueError("padding only supported after the last row")
      return self.S
    return self.n_vis + self.text_real

  @property
  def padded(self) -> bool:
    return self.kv_len != self.S

  def attn_flops(self) -> float:
    """4*B*H*Sq*Skv_valid*D (QK^T + PV, 2 flop per MAC)."""
    return 4.0 * self.B * self.H * self.S * self.kv_len * self.D

  def prologue_bytes(self) -> float:
    """Read q, k and write q, k (bf16), plus the two fp32 weight vectors."""
    return 8.0 * self.B * self.S * self.H * self.D + 8.0 * self.D

  def positions(self) -> np.ndarray:
    """int32 (S, 3) positions over (t, h, w)."""
    t, hh, ww = self.grid
    tt, yy, xx = np.meshgrid(np.arange(t), np.arange(hh), np.arange(ww),
                             indexing="ij")
    vis = np.stack([tt.ravel(), yy.ravel(), xx.ravel()], 1)
    txt = np.zeros((self.text, 3), np.int64)
    pos = np.concatenate([txt, vis] if self.text_first else [vis, txt], 0)
    return pos.astype(np.int32)

  def inputs(self, device="cpu", seq_rows=None):
    """Seeded inputs: dict of q, k (B,S,H,D), v (B,H,S,D), wq, wk, hs.

    ``seq_rows`` keeps only the first rows of the sequence (for small CPU
    checks at the real H, D and RoPE split); padding is then not applied.
    Tensors are drawn in float32 on ``device`` and cast to ``in_dtype``.
    """
    s = self.S if seq_rows is None else int(seq_rows)
    def normal(seed, shape):
      g = torch.Generator(device=device).manual_seed(seed)
      return torch.randn(shape, generator=g, device=device,
                         dtype=torch.float32)
    b, h, d = self.B, self.H, self.D
    out = {
        "q": normal(0, (b, s, h, d)).to(self.in_dtype),
        "k": normal(1, (b, s, h, d)).to(self.in_dtype),
        "v": normal(2, (b, h, s, d)).to(self.in_dtype),
    }
    g = torch.Generator(device="cpu").manual_seed(3)
    w = 1.0 + 0.02 * torch.randn((2, d), generator=g, dtype=torch.float32)
    out["wq"], out["wk"] = w[0].to(device), w[1].to(device)
    if self.head_scale:
      g = torch.Generator(device="cpu").manual_seed(4)
      out["hs"] = (0.5 + torch.rand((h,), generator=g,
                                    dtype=torch.float32)).to(device)
    else:
      out["hs"] = None
    if seq_rows is None and self.padded:
      # padded values are zero, as the reference's callers make them
      out["v"][:, :, self.kv_len:] = 0
    out["pos"] = torch.from_numpy(self.positions()[:s].copy()).to(device)
    return out


WORKLOADS = {
    # plumbing, fp32 inputs, 1D RoPE over all 64 channels
    "P": Workload("P", B=1, H=8, D=64, grid=(1024, 1, 1), axis_dims=(64, 0, 0),
                  in_dtype=torch.float32, desc="plumbing, 1D RoPE"),
    # image 1024^2, CFG pair, 300 of 512 text rows real
    "I1": Workload("I1", B=2, H=24, D=128, grid=(1, 64, 64), text=512,
                   text_real=300, axis_dims=(0, 64, 64),
                   desc="image 1024x1024, CFG pair"),
    # image 2048^2, 137 of 512 text rows real
    "I2": Workload("I2", B=1, H=24, D=128, grid=(1, 128, 128), text=512,
                   text_real=137, axis_dims=(0, 64, 64),
                   desc="image 2048x2048"),
    # video 480x832x121, text rows first, 3D RoPE 44/42/42
    "V4": Workload("V4", B=1, H=40, D=128, grid=(31, 30, 52), text=512,
                   text_real=512, text_first=True, axis_dims=(44, 42, 42),
                   desc="video 480x832x121"),
    # video 768x1344x345 head shard (5 of 40 heads), per-head scale
    "V7": Workload("V7", B=1, H=5, D=128, grid=(87, 48, 84),
                   axis_dims=(44, 42, 42), head_scale=True,
                   desc="video 768x1344x345 head shard"),
}

MFMA_BF16_DENSE_PEAK = 2.5e15  # MI355X dense bf16 MFMA, FLOP/s
HBM_PEAK = 8.0e12              # MI355X HBM3E, B/s
