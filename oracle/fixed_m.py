"""Fixed-m bound oracle (test infrastructure; see ``oracle/__init__.py``).

Restates ``diffusers_tpu/kernels/fixed_m_bound.py:57-118``: per head, the
Cauchy-Schwarz bound ``max_{b,s}|q_scaled| * max_{b,s}|k|`` on any logit
(in log2 units when ``q_scaled`` carries ``scale*log2(e)``), its integral
ceiling used as the kernel's ``m`` and the eligibility flag
``bound <= gate``.
"""
from __future__ import annotations

import numpy as np

LOG2_E = 1.44269504            # fixed_m_bound.py:37
FIXED_M_RECENTER = 88.0        # fixed_m_bound.py:42
FIXED_M_SAFE_BOUND = 213.0     # fixed_m_bound.py:47
FIXED_M_RING_SAFE_BOUND = FIXED_M_SAFE_BOUND / 2.0  # fixed_m_bound.py:54


def max_row_norm_per_head(x):
  """``(heads,)`` max over (B, S) of the L2 row norm (fixed_m_bound.py:57-73)."""
  x = np.asarray(x, np.float64)
  return np.sqrt((x * x).sum(-1)).max(axis=(0, 2))


def fixed_m_operands(q_scaled, k, gate=FIXED_M_SAFE_BOUND):
  """``(2, heads)``: row 0 ceil(bound), row 1 flag (fixed_m_bound.py:98-118)."""
  bound = max_row_norm_per_head(q_scaled) * max_row_norm_per_head(k)
  return np.stack([np.ceil(bound), (bound <= gate).astype(np.float64)])


def bf16_round(x):
  """Round to the nearest bfloat16 (ties to even), returned as float64.

  The float32 bit pattern keeps its top 16 bits after adding the rounding
  bias 0x7fff + lsb, the standard round-to-nearest-even on the dropped half.
  (Inputs are finite.)"""
  b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
  b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
  return b.astype(np.uint32).view(np.float32).astype(np.float64)


def smooth_keys(k, kv_len=None):
  """Key smoothing as models/minimax_h3/jax_server.py:271-289 does it on
  bf16 keys ``[B, H, S, D]``: the mean over rows ``[0, kv_len)`` (all rows
  when ``kv_len`` is None), cast to bf16, subtracted in bf16 (exact
  difference rounded once), rows at or past ``kv_len`` zero.  The mean is
  taken in float64 here (the reference sums in float32: the two round to
  the same bf16 except within float32 error of a rounding boundary)."""
  k = np.asarray(k, np.float64)
  n = k.shape[2] if kv_len is None else int(kv_len)
  mean = bf16_round(k[:, :, :n].mean(axis=2, keepdims=True))
  out = bf16_round(k - mean)
  out[:, :, n:] = 0.0
  return out, mean


def max_abs_logit_bruteforce(q, k, factor, stride=1):
  """``(heads,)`` max over query rows ``0, stride, ...`` and every key of
  ``|bf16(factor * q) . k|`` by explicit loops over rows (test
  infrastructure for ``sampled_max_abs_logit``, kernels/fixed_m_bound.py:
  169-286).  q, k: ``[B, H, S, D]`` (k already bf16-valued)."""
  q = np.asarray(q, np.float64)
  k = np.asarray(k, np.float64)
  b, h, s, _ = q.shape
  best = np.zeros(h)
  for bb in range(b):
    for hh in range(h):
      for i in range(0, s, stride):
        qs = bf16_round(np.float32(factor) * q[bb, hh, i].astype(np.float32))
        for j in range(k.shape[2]):
          best[hh] = max(best[hh], abs(float(np.dot(qs, k[bb, hh, j]))))
  return best
