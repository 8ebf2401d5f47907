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
