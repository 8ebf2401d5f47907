"""Key smoothing, ``k - mean_S(k)``: the caller contract of fixed-m
(gfx950 kernel ``dt_smooth_keys``).

The reference subtracts the per-(batch, head) channel mean of the keys
before its fixed-m attention (kernels/mesh_attention.py:234-237,
backends/ours_splash_tt.py:136-137), over the real rows only when the
sequence is padded, zeroing the padded rows
(models/minimax_h3/jax_server.py:271-289): the mean in float32, cast to the
key dtype, subtracted.  Softmax attention is unchanged by it; fixed-m's
no-flush gate rests on it (zero-mean keys make every row's mean logit 0,
so rowmax >= 0).

``smooth_keys`` does it in one read for the mean and one read + write for
the subtraction, and can return the smoothed keys' per-head max row norm
from the same pass, which is the key half of the fixed-m bound
(kernels/fixed_m_bound.py:57-73).
"""
from __future__ import annotations

import torch

from .. import _lib


def _torch_smooth(key, n):
  """Same arithmetic with torch ops, for head dims the kernel does not
  cover and non-bf16 keys."""
  mean = key[:, :, :n].float().mean(dim=2, keepdim=True).to(key.dtype)
  ks = key - mean
  if n < key.shape[2]:
    ks[:, :, n:] = 0
  return ks


def smooth_keys(key: torch.Tensor, kv_len=None, *, out=None,
                norms: bool = False):
  """``key`` ``(B, H, S, D)`` minus its mean over rows ``[0, kv_len)``.

  Rows at or past ``kv_len`` come out zero.  ``out``: optional bf16
  destination of the same shape (may be ``key`` itself).  With
  ``norms=True`` returns ``(ks, kn)``, ``kn`` the ``(H,)`` float32 max over
  (batch, row) of ``||ks[b, h, s]||``.
  """
  if not key.is_cuda:
    raise ValueError("key must be on the GPU; the gfx950 kernel has no CPU "
                     "path")
  if key.dim() != 4:
    raise ValueError(f"key must be (B, H, S, D), got {tuple(key.shape)}")
  b, h, s, d = key.shape
  n, n_dev = _lib.length_arg(kv_len, s, key.device, batch=b)
  kernel_ok = (key.dtype == torch.bfloat16 and d in (64, 128, 256) and
               key.stride(-1) == 1 and all(t % 8 == 0 for t in key.stride()[:3])
               and key.data_ptr() % 16 == 0)
  if not kernel_ok:
    if n_dev is not None:
      raise NotImplementedError("a device kv_len needs a bf16 key with head "
                                "dim 64, 128 or 256")
    ks = _torch_smooth(key, n)
    if out is not None:
      out.copy_(ks)
      ks = out
    if norms:
      from .fixed_m_bound import max_row_norm_per_head
      return ks, max_row_norm_per_head(ks.to(torch.bfloat16))
    return ks
  if out is None:
    out = torch.empty_like(key, memory_format=torch.contiguous_format)
  elif (out.shape != key.shape or out.dtype != torch.bfloat16 or
        out.device != key.device or out.stride(-1) != 1 or
        any(t % 8 for t in out.stride()[:3]) or out.data_ptr() % 16):
    raise ValueError("out must be a bf16 (B, H, S, D) tensor on key's device "
                     "with a contiguous last axis and 8-element strides")
  lib = _lib.load()
  with torch.cuda.device(key.device):
    nbytes = lib.dt_smooth_keys_workspace_bytes(b, h, s, d,
                                                0 if n_dev is not None else n)
    ws = torch.empty((nbytes + 3) // 4, device=key.device, dtype=torch.float32)
    kn = torch.zeros(h, device=key.device, dtype=torch.float32) if norms \
        else None
    rc = lib.dt_smooth_keys(
        key.data_ptr(), out.data_ptr(), b, h, s, d,
        _lib.i64_array(*key.stride()[:3]), _lib.i64_array(*out.stride()[:3]),
        n, _lib.ptr(n_dev), None if kn is None else kn.data_ptr(),
        ws.data_ptr(), nbytes,
        torch.cuda.current_stream(key.device).cuda_stream)
  _lib.check("dt_smooth_keys", rc)
  return (out, kn) if norms else out
