"""QK-RMSNorm + RoPE oracle (test infrastructure; see ``oracle/__init__.py``).

RMSNorm: ``y = x * rsqrt(mean_D(x^2) + eps) * w`` with the reduction in
float32-or-wider, as ``models/minimax_h3/jax_dit.py:191-195`` (and the Qwen
``RMSNorm`` ``models/qwen_image_21/jax_dit.py:188-192``, MOSS ``_rms``
``models/moss_image/jax_dit.py:126-129``).  The reference variants differ
only in where they round to bf16; this oracle rounds nowhere (float64).

RoPE: the leading ``rotary = sum(axis_dims)`` channels rotate, the rest pass
through (``models/minimax_h3/jax_dit.py:251-262``).  Rotation pair ``j`` in
``[0, rotary/2)`` belongs to axis ``a`` (axes take ``axis_dims[a]/2``
consecutive pairs) with frequency ``theta^(-2i/axis_dims[a])`` for its index
``i`` inside the axis; its angle is ``pos[s, a] * freq``.  With
``axis_dims=(32,32,32)`` this is exactly H3's ``rope_angles``
(``jax_dit.py:603-617``: one inv_freq of 16 entries shared by t,h,w, 96
rotated channels); with ``(16,56,56)`` in interleaved mode it is Qwen's
``axes_dims_rope`` table (``qwen_image_21/jax_dit.py:515,585``).

Conventions:

* ``"half"``  rotate-half: pair j = channels (j, j + rotary/2);
  ``out = x*cos + cat(-x2, x1)*sin`` (H3 ``apply_rope`` :251-262, MOSS
  ``_rotate`` moss_image/jax_dit.py:136-142).
* ``"pair"``  interleaved complex pairs: pair j = channels (2j, 2j+1),
  multiplied by ``exp(i*angle)`` (Qwen ``apply_rope`` :214-220).
"""
from __future__ import annotations

import numpy as np


def rms_norm_f64(x, w, eps):
  """``x * rsqrt(mean(x^2, -1) + eps) * w`` in float64 (jax_dit.py:191-195)."""
  x = np.asarray(x, np.float64)
  r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
  return x * r * np.asarray(w, np.float64)


def rope_freqs(axis_dims, theta):
  """Per-pair frequency, length ``sum(axis_dims)//2`` (float64)."""
  out = []
  for dim in axis_dims:
    if dim % 2:
      raise ValueError(f"axis dim {dim} must be even")
    i = np.arange(dim // 2, dtype=np.float64)
    out.append(theta ** (-2.0 * i / dim))
  return np.concatenate(out) if out else np.zeros(0)


def rope_pair_axis(axis_dims):
  """Axis index of every rotation pair."""
  return np.concatenate([np.full(d // 2, a, np.int64)
                         for a, d in enumerate(axis_dims)])


def rope_angles_f64(pos, axis_dims, theta):
  """``(S, rotary/2)`` angles from integer positions ``pos`` ``(S, 3)``."""
  pos = np.asarray(pos, np.float64)
  return pos[:, rope_pair_axis(axis_dims)] * rope_freqs(axis_dims, theta)


def apply_rope_f64(x, angles, mode):
  """Rotate ``x`` ``[..., S, D]`` (sequence on axis -2) by ``angles``.

  ``angles`` is ``(S, rotary/2)``; channels past ``rotary`` pass through.
  """
  x = np.asarray(x, np.float64)
  half = angles.shape[-1]
  rot = 2 * half
  c, s = np.cos(angles), np.sin(angles)
  out = x.copy()
  if mode == "half":
    x1, x2 = x[..., :half], x[..., half:rot]
    out[..., :half] = x1 * c - x2 * s
    out[..., half:rot] = x2 * c + x1 * s
  elif mode == "pair":
    x0, x1 = x[..., 0:rot:2], x[..., 1:rot:2]
    out[..., 0:rot:2] = x0 * c - x1 * s
    out[..., 1:rot:2] = x0 * s + x1 * c
  else:
    raise ValueError(mode)
  return out


def apply_rope_table_f64(x, cos, sin, mode):
  """Rotate ``x`` ``[B, S, H, D]`` by per-token tables.

  ``cos``/``sin`` are ``(S, half)`` or ``(B, S, half)``: the cosine and sine
  of rotation pair ``j`` at token ``(b, s)``; pairs as in
  ``apply_rope_f64``, channels past ``2*half`` pass through.  This is the
  general form both reference table conventions reduce to (H3
  ``apply_rope`` jax_dit.py:251-262 with repeated halves, MOSS ``_rotate``
  moss_image/jax_dit.py:136-142).
  """
  x = np.asarray(x, np.float64)
  c = np.asarray(cos, np.float64)
  s = np.asarray(sin, np.float64)
  if c.ndim == 2:
    c, s = c[None], s[None]
  c, s = c[:, :, None, :], s[:, :, None, :]     # broadcast over heads
  half = c.shape[-1]
  rot = 2 * half
  out = x.copy()
  if mode == "half":
    x1, x2 = x[..., :half], x[..., half:rot]
    out[..., :half] = x1 * c - x2 * s
    out[..., half:rot] = x2 * c + x1 * s
  elif mode == "pair":
    x0, x1 = x[..., 0:rot:2], x[..., 1:rot:2]
    out[..., 0:rot:2] = x0 * c - x1 * s
    out[..., 1:rot:2] = x0 * s + x1 * c
  else:
    raise ValueError(mode)
  return out


def h3_apply_rope_f64(x, cos, sin):
  """H3's ``apply_rope`` (models/minimax_h3/jax_dit.py:251-262) as written:
  ``x`` ``[B, S, H, D]``, ``cos``/``sin`` ``(S, rotary)``; the leading
  ``rotary`` channels become ``rotated*cos + cat(-x2, x1)*sin``."""
  x = np.asarray(x, np.float64)
  rot = cos.shape[-1]
  r, rest = x[..., :rot], x[..., rot:]
  c = np.asarray(cos, np.float64)[None, :, None, :]
  s = np.asarray(sin, np.float64)[None, :, None, :]
  x1, x2 = r[..., :rot // 2], r[..., rot // 2:]
  turned = np.concatenate([-x2, x1], -1)
  return np.concatenate([r * c + turned * s, rest], -1)


def moss_rotate_f64(x, rope):
  """MOSS's ``_rotate`` (models/moss_image/jax_dit.py:136-142) as written:
  ``x`` ``[B, S, H, D]``, ``rope`` ``[B, S, D]`` = ``[sin | cos]`` halves,
  each repeated over both halves of the head."""
  x = np.asarray(x, np.float64)
  rope = np.asarray(rope, np.float64)
  half = rope.shape[-1] // 2
  sin, cos = rope[..., :half], rope[..., half:]
  sin = np.concatenate([sin, sin], -1)[:, :, None]
  cos = np.concatenate([cos, cos], -1)[:, :, None]
  a, b = x[..., :x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
  return x * cos + np.concatenate([-b, a], -1) * sin


def qk_norm_rope_table_f64(x, w, eps, cos, sin, mode, *, head_scale=None,
                           valid_len=None):
  """``qk_norm_rope_f64`` with the rotation from per-token tables."""
  y = apply_rope_table_f64(rms_norm_f64(x, w, eps), cos, sin, mode)
  if head_scale is not None:
    y = y * np.asarray(head_scale, np.float64)[None, None, :, None]
  if valid_len is not None:
    y[:, valid_len:] = 0.0
  return y


def qk_norm_rope_f64(x, w, eps, pos, axis_dims, theta, mode, *,
                     head_scale=None, valid_len=None):
  """The fused prologue on one tensor ``[B, S, H, D]`` -> ``[B, S, H, D]``.

  RMSNorm (jax_dit.py:362-363) then RoPE (:365-366); optional per-head
  factor (folded after the rotation, a per-head scalar commutes with it);
  rows at or past ``valid_len`` zeroed (jax_dit.py:367-381).
  """
  y = rms_norm_f64(x, w, eps)
  if mode != "none":
    ang = rope_angles_f64(pos, axis_dims, theta)  # (S, half)
    y = np.swapaxes(apply_rope_f64(np.swapaxes(y, 1, 2), ang, mode), 1, 2)
  if head_scale is not None:
    y = y * np.asarray(head_scale, np.float64)[None, None, :, None]
  if valid_len is not None:
    y[:, valid_len:] = 0.0
  return y
