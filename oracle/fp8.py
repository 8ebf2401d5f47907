"""E4M3 saturating cast oracle (test infrastructure; see ``oracle/__init__.py``).

Restates ``diffusers_tpu/kernels/fp8_cast.py:28-39``: clip to +-E4M3_MAX
(448, ``kernels/e4m3.py:25``), then round to the nearest OCP e4m3fn value,
ties to even.  The format is decoded from its definition (1 sign, 4 exponent
bits with bias 7, 3 mantissa bits; exponent field 0 is subnormal; only
S.1111.111 is NaN, so 448 = 0x7E is the largest finite value) rather than
taken from a library.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0  # kernels/e4m3.py:25


def decode_e4m3(code):
  """Value of each e4m3fn byte (NaN for 0x7F / 0xFF)."""
  code = np.asarray(code, np.int64)
  sign = np.where(code & 0x80, -1.0, 1.0)
  exp = (code >> 3) & 0xF
  man = code & 0x7
  val = np.where(exp == 0, man / 8.0 * 2.0**-6,
                 (1.0 + man / 8.0) * 2.0**(exp - 7.0))
  val = np.where((code & 0x7F) == 0x7F, np.nan, val)
  return sign * val


_POS = decode_e4m3(np.arange(0x7F))  # finite non-negative codes, ascending


def quantize_e4m3(x):
  """Codes (uint8) of ``clip(x, -448, 448)`` rounded to nearest, ties even."""
  x = np.asarray(x, np.float64)
  a = np.minimum(np.abs(x), E4M3_MAX)
  hi = np.clip(np.searchsorted(_POS, a), 0, len(_POS) - 1)
  lo = np.maximum(hi - 1, 0)
  dlo, dhi = a - _POS[lo], _POS[hi] - a
  pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi,
                                          np.where(lo % 2 == 0, lo, hi)))
  return (pick | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)


def e4m3_round(x):
  """``x`` after the saturating E4M3 cast, as float64."""
  return decode_e4m3(quantize_e4m3(x))
