"""Shared helpers of the GPU parity tests (the oracle is the checker)."""
import numpy as np
import torch

# north-star tolerances (bf16 attention vs an fp32-or-wider softmax oracle)
ATTN_MAX_ABS = 2e-2
ATTN_MEAN_ABS = 2e-3
PROLOGUE_MAX_ABS = 1e-2


def to64(t):
  return t.detach().float().cpu().numpy().astype(np.float64)


def seeded(shape, seed, device="cuda", dtype=torch.bfloat16):
  g = torch.Generator(device="cpu").manual_seed(seed)
  return torch.randn(shape, generator=g, dtype=torch.float32).to(
      device=device, dtype=dtype)


def assert_attn_close(got, want, what=""):
  got = np.asarray(got, np.float64)
  err = np.abs(got - want)
  assert np.isfinite(got).all(), f"{what}: non-finite output"
  assert err.max() <= ATTN_MAX_ABS, f"{what}: max-abs {err.max():.3g}"
  assert err.mean() <= ATTN_MEAN_ABS, f"{what}: mean-abs {err.mean():.3g}"
  return float(err.max()), float(err.mean())


def banner(msg):
  print(f"[gpu-case] {msg}", flush=True)
