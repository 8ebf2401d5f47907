"""Saturating E4M3 cast — mirror of ``diffusers_tpu/kernels/fp8_cast.py``.

``quantize_saturating`` clamps to +-448 (``E4M3_MAX``, kernels/e4m3.py:25)
and casts to ``float8_e4m3fn`` (kernels/fp8_cast.py:28-39) on the GPU with
the gfx950 kernel ``dt_quantize_e4m3`` (one HBM pass, 2 bytes in and 1 byte
out per element).  Inputs are cast to bf16 first; the result is a
contiguous ``torch.float8_e4m3fn`` tensor of the same shape.
"""
from __future__ import annotations

import torch

from .. import _lib

E4M3_MAX = 448.0  # kernels/e4m3.py:25


def quantize_saturating(x: torch.Tensor, *, factor: float = 1.0,
                        out: torch.Tensor | None = None) -> torch.Tensor:
  """``e4m3fn(clamp(bf16(factor * x), -448, 448))`` of a 4-D GPU tensor.

  The leading three axes are any (b, h, s) indexing; the last axis (a
  multiple of 8) is contiguous in the output.
  """
  if not isinstance(x, torch.Tensor) or x.dim() != 4:
    raise ValueError("x must be a 4-D torch.Tensor")
  if not x.is_cuda:
    raise ValueError("x must be on the GPU; the gfx950 kernel has no CPU path")
  if x.shape[-1] % 8:
    raise NotImplementedError(f"last dim {x.shape[-1]} not a multiple of 8")
  if x.dtype != torch.bfloat16:
    x = x.to(torch.bfloat16)
  if x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:3]) or \
     x.data_ptr() % 16:
    x = x.contiguous()
  if out is None:
    out = torch.empty(x.shape, device=x.device, dtype=torch.float8_e4m3fn)
  elif out.shape != x.shape or out.dtype != torch.float8_e4m3fn or \
      out.stride(-1) != 1 or out.device != x.device:
    raise ValueError("out must be a float8_e4m3fn GPU tensor of x's shape "
                     "with a contiguous last axis")
  b, h, s, d = x.shape
  lib = _lib.load()
  with torch.cuda.device(x.device):
    rc = lib.dt_quantize_e4m3(
        x.data_ptr(), out.data_ptr(), b, h, s, d,
        _lib.i64_array(*x.stride()[:3]), _lib.i64_array(*out.stride()[:3]),
        float(factor), torch.cuda.current_stream(x.device).cuda_stream)
  _lib.check("dt_quantize_e4m3", rc)
  return out
