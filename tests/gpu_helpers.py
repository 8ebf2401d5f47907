"""Shared helpers of the GPU parity tests (the oracle is the checker)."""
import numpy as np
import torch

# north-star tolerances (bf16 attention vs an fp32-or-wider softmax oracle)
ATTN_MAX_ABS = 2e-2
ATTN_MEAN_ABS = 2e-3
PROLOGUE_MAX_ABS = 1e-2


def bf16_round(x):
  """float64 values rounded to the nearest bf16 (the prologue's output type,
  as the reference's), returned as float64."""
  t = torch.from_numpy(np.ascontiguousarray(x, np.float64)).float()
  return t.to(torch.bfloat16).double().numpy()


def bf16_ulp(x):
  """Spacing of bf16 values at |x| (8 significant bits; normal range)."""
  x = np.abs(np.asarray(x, np.float64))
  _, e = np.frexp(np.where(x > 0, x, 1.0))   # x = f * 2^e, f in [0.5, 1)
  return np.where(x > 0, np.ldexp(1.0, e - 8), np.ldexp(1.0, -133))


def prologue_errors(got, want):
  """Errors of the prologue's bf16 output ``got`` against the float64
  oracle ``want``:

  * ``kernel``: how far ``want`` lies outside the interval of reals that
    round to ``got`` (half a bf16 step either side), i.e. the error of the
    kernel's own arithmetic with the output's final rounding taken out.  A
    correctly rounded result has 0.
  * ``steps``: the largest distance between ``got`` and ``bf16(want)`` in
    bf16 steps (0: the correctly rounded value; 1: its neighbour, where the
    kernel's float32 arithmetic lands on the other side of a rounding
    boundary).
  * ``full``: max |got - want| (the output rounding included).
  * ``exact``: the share of elements equal to ``bf16(want)``.
  """
  got = np.asarray(got, np.float64)
  want = np.asarray(want, np.float64)
  ref = bf16_round(want)
  ulp = bf16_ulp(got)
  excess = np.maximum(np.abs(got - want) - 0.5 * ulp, 0.0)
  steps = np.abs(got - ref) / np.maximum(bf16_ulp(ref), 1e-300)
  return {"kernel": float(excess.max(initial=0.0)),
          "steps": float(steps.max(initial=0.0)),
          "full": float(np.abs(got - want).max(initial=0.0)),
          "vs_bf16": float(np.abs(got - ref).max(initial=0.0)),
          "exact": float((got == ref).mean()) if got.size else 1.0}


def assert_prologue_close(got, want, what=""):
  """The prologue's bf16 output against the float64 oracle: the kernel's
  arithmetic error (output rounding taken out) within the north-star
  1e-2 max-abs.  Returns the errors of ``prologue_errors`` (the others are
  reported, not bounded: near zero, where a rotation cancels, a float32
  error far below 1e-2 is many bf16 steps)."""
  e = prologue_errors(got, want)
  assert np.isfinite(np.asarray(got)).all(), f"{what}: non-finite output"
  assert e["kernel"] <= PROLOGUE_MAX_ABS, \
      f"{what}: arithmetic error {e['kernel']:.3g} beyond the output " \
      f"rounding ({e['exact']:.4f} correctly rounded)"
  return e


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
