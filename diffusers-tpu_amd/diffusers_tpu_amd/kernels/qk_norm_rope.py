"""Fused QK-RMSNorm + RoPE prologue (gfx950 HIP kernel ``dt_qk_norm_rope``).

Replaces the per-layer stage every reference DiT attention block runs on q
and k right before attention: RMSNorm (models/minimax_h3/jax_dit.py:191-195,
applied :362-363), RoPE (apply_rope :251-262, applied :365-366), zeroing of
padded rows (:367-381) and the ``(B,S,H,D) -> (B,H,S,D)`` transpose (:388),
in one pass that reads q, k once and writes them once.

RoPE is described by a ``RopeSpec``: a convention (``"half"`` rotate-half as
H3/MOSS, ``"pair"`` interleaved complex pairs as Qwen), integer positions per
token ``(S, 3)`` over (t, h, w) axes, the channel count each axis owns and
``theta``.  The reference's H3 table (``rope_angles``, jax_dit.py:603-617,
rope_freq_dim=16) is ``RopeSpec("half", pos, (32, 32, 32), 1e4)``; rows the
reference gives the identity rotation (text / padding, jax_dit.py:727-731)
take position (0, 0, 0).

Models that hand the attention block ready-made cos/sin tables instead of
positions use a ``RopeTable`` (kernel ``dt_qk_norm_rope_table``): H3's
``apply_rope(x, cos, sin)`` with ``(S, rotary)`` tables whose halves repeat
(``RopeTable.from_cos_sin``) and MOSS's ``_rotate(x, rope)`` with a
``(B, S, D)`` ``[sin | cos]`` tensor (``RopeTable.from_sin_cos_rows``,
moss_image/jax_dit.py:136-142).

Arithmetic is fp32 throughout with one rounding to bf16 at the end; the
reference variants round at different points (H3 after the weight, MOSS
before it, Qwen returns fp32), so results agree to bf16 rounding.
"""
from __future__ import annotations

import dataclasses

import torch

from .. import _lib

_MODES = {"none": _lib.ROPE_NONE, "half": _lib.ROPE_HALF,
          "pair": _lib.ROPE_PAIR}


@dataclasses.dataclass
class RopeSpec:
  """RoPE description.

  Attributes:
    mode: ``"half"`` (rotate-half) or ``"pair"`` (interleaved pairs).
    positions: int32 ``(S, 3)`` tensor of (t, h, w) positions on the GPU
      (unused axes 0).
    axis_dims: channels rotated per axis; their sum is the rotary width.
    theta: base frequency.
  """
  mode: str
  positions: torch.Tensor
  axis_dims: tuple = (0, 0, 0)
  theta: float = 10000.0


@dataclasses.dataclass
class RopeTable:
  """RoPE given as per-token cos/sin of each rotation pair.

  Attributes:
    mode: ``"half"`` (pair j = channels (j, j + rot/2)) or ``"pair"``
      (pair j = channels (2j, 2j + 1)).
    cos, sin: ``(S, rot/2)`` or ``(B, S, rot/2)`` tensors on the GPU (any
      float dtype; float32 views are used in place).  Channels past ``rot``
      pass through.
  """
  mode: str
  cos: torch.Tensor
  sin: torch.Tensor

  @classmethod
  def from_cos_sin(cls, cos, sin, mode="half"):
    """H3's ``apply_rope`` tables (models/minimax_h3/jax_dit.py:251-262):
    ``(S, rotary)`` cos and sin whose two halves are equal, as
    ``rope_angles`` builds them (jax_dit.py:603-617).  The kernel reads the
    first half; ``check_halves`` verifies the second repeats it."""
    half = cos.shape[-1] // 2
    if mode == "half":
      return cls(mode, cos[..., :half], sin[..., :half])
    return cls(mode, cos, sin)

  @classmethod
  def from_sin_cos_rows(cls, rope):
    """MOSS's ``rope`` operand ``(B, S, D)`` = ``[sin | cos]`` halves of
    D/2, each applied to both halves of the head (moss_image/jax_dit.py:
    136-142): a rotate-half over all D channels."""
    half = rope.shape[-1] // 2
    return cls("half", rope[..., half:], rope[..., :half])


def check_halves(cos, sin):
  """True when ``(.., rotary)`` cos/sin repeat their first half, the form
  ``RopeTable.from_cos_sin`` relies on (synchronises with the GPU)."""
  h = cos.shape[-1] // 2
  return bool(torch.equal(cos[..., :h], cos[..., h:]) and
              torch.equal(sin[..., :h], sin[..., h:]))


def _table_operand(t, b, s, dev, name):
  """fp32 view (or copy) of a table and its (batch, seq) strides."""
  t = t.to(device=dev, dtype=torch.float32)
  if t.dim() == 2:
    t = t.unsqueeze(0)
  if t.dim() != 3 or t.shape[1] != s or t.shape[0] not in (1, b):
    raise ValueError(f"rope {name} must be (S, n) or (B, S, n) with S={s}, "
                     f"B={b}; got {tuple(t.shape)}")
  if t.stride(-1) != 1:
    t = t.contiguous()
  sb = 0 if t.shape[0] == 1 else t.stride(0)
  return t, sb, t.stride(1)


def _prep(t, name, keep_f32=False):
  """bf16 (or, with ``keep_f32``, fp32 kept as it is) with a contiguous
  last axis and 8-element-aligned strides."""
  if not t.is_cuda:
    raise ValueError(f"{name} must be on the GPU; the gfx950 kernel has no CPU "
                     "path")
  if t.dim() != 4:
    raise ValueError(f"{name} must be [B, S, H, D], got {tuple(t.shape)}")
  if t.dtype != torch.bfloat16 and not (keep_f32 and t.dtype == torch.float32):
    t = t.to(torch.bfloat16)
  if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or \
     t.data_ptr() % 16:
    t = t.contiguous()
  return t


def qk_norm_rope(q, k, wq, wk, *, eps=1e-6, rope=None, q_head_scale=None,
                 valid_len=None, out_layout="bhsd", out=None):
  """RMSNorm + RoPE on q and k in one kernel.

  Args:
    q, k: ``(B, S, H, D)`` GPU tensors: bf16, or fp32 (both; read as fp32
      by the kernel); other dtypes converted to bf16.  Any strides with a contiguous last
      axis, e.g. a view of a fused projection.
    wq, wk: ``(D,)`` RMSNorm weights (float32 after conversion).
    eps: RMSNorm epsilon (H3 1e-5, Qwen/MOSS 1e-6).
    rope: a ``RopeSpec`` (positions), a ``RopeTable`` (cos/sin per token)
      or ``None`` for RMSNorm only.
    q_head_scale: optional ``(H,)`` factor applied to q after rotation.
    valid_len: rows ``s >= valid_len`` come out as zeros (padded queries and
      keys, jax_dit.py:367-381); ``None`` keeps every row.  An int, or a
      one-element integer tensor on the GPU, which the kernel reads when it
      runs (no host sync; a captured graph serves every length; a value
      <= 0 zeroes every row).  Per-sample lengths: a B-element GPU tensor or
      a host sequence of B ints, batch element b zeroed from its own
      length.
    out_layout: ``"bhsd"`` (what ``attention`` takes) or ``"bshd"``.
    out: optional preallocated ``(q_out, k_out)`` in ``out_layout``.

  Returns:
    ``(q_out, k_out)`` bf16 in ``out_layout``.
  """
  # fp32 q and k are read as fp32 by the kernel (dt_qk_norm_rope_f32,
  # dt_qk_norm_rope_table_f32); everything else is taken as bf16
  f32 = q.dtype == torch.float32 and k.dtype == torch.float32
  q = _prep(q, "q", f32)
  k = _prep(k, "k", f32)
  if q.device != k.device:
    raise ValueError(f"k is on {k.device}, q on {q.device}")
  if q.shape != k.shape:
    raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} differ")
  if q.stride() != k.stride():
    k = k.contiguous()
    q = q.contiguous()
  b, s, h, d = q.shape
  dev = q.device
  wq = wq.to(device=dev, dtype=torch.float32).contiguous()
  wk = wk.to(device=dev, dtype=torch.float32).contiguous()
  if wq.shape != (d,) or wk.shape != (d,):
    raise ValueError(f"norm weights must be ({d},)")
  hs = None
  if q_head_scale is not None:
    hs = q_head_scale.to(device=dev, dtype=torch.float32).contiguous()
    if hs.shape != (h,):
      raise ValueError(f"q_head_scale must be ({h},)")
  if out_layout == "bhsd":
    shape = (b, h, s, d)
  elif out_layout == "bshd":
    shape = (b, s, h, d)
  else:
    raise ValueError(f"out_layout {out_layout!r}")
  if out is None:
    qo = torch.empty(shape, device=dev, dtype=torch.bfloat16)
    ko = torch.empty(shape, device=dev, dtype=torch.bfloat16)
  else:
    qo, ko = out
    if qo.shape != shape or ko.shape != shape or qo.stride() != ko.stride():
      raise ValueError("out tensors have the wrong shape or strides")
    if any(t.dtype != torch.bfloat16 or t.device != dev or t.stride(-1) != 1
           for t in (qo, ko)):
      raise ValueError("out tensors must be bf16 on q's device with a "
                       "contiguous last axis")
  if out_layout == "bhsd":
    ostr = (qo.stride(0), qo.stride(2), qo.stride(1))
  else:
    ostr = qo.stride()[:3]
  if valid_len is None:
    vl, vl_dev = -1, None
  else:
    vl, vl_dev = _lib.length_arg(valid_len, s, dev, "valid_len", batch=b)
  lib = _lib.load()
  stream = torch.cuda.current_stream(dev).cuda_stream
  if isinstance(rope, RopeTable):
    if rope.mode not in ("half", "pair"):
      raise ValueError(f"rope table mode {rope.mode!r}")
    if rope.cos.shape != rope.sin.shape:
      raise ValueError(f"cos {tuple(rope.cos.shape)} and sin "
                       f"{tuple(rope.sin.shape)} differ")
    cos, sb, ss = _table_operand(rope.cos, b, s, dev, "cos")
    sin, sb2, ss2 = _table_operand(rope.sin, b, s, dev, "sin")
    if (sb, ss) != (sb2, ss2):      # one stride pair serves both tables
      n = max(cos.shape[0], sin.shape[0])
      cos = cos.expand(n, -1, -1).contiguous()
      sin = sin.expand(n, -1, -1).contiguous()
      sb, ss = (0 if n == 1 else cos.stride(0)), cos.stride(1)
    rot = 2 * cos.shape[-1]
    fn = lib.dt_qk_norm_rope_table_f32 if f32 else lib.dt_qk_norm_rope_table
    with torch.cuda.device(dev):
      rc = fn(
          q.data_ptr(), k.data_ptr(), qo.data_ptr(), ko.data_ptr(), b, s, h,
          d, _lib.strides3(q.stride()), _lib.strides3(ostr),
          wq.data_ptr(), wk.data_ptr(), float(eps),
          None if hs is None else hs.data_ptr(), _MODES[rope.mode],
          cos.data_ptr(), sin.data_ptr(), _lib.i64_array(sb, ss), rot, vl,
          _lib.ptr(vl_dev), stream)
    _lib.check("dt_qk_norm_rope_table_f32" if f32 else
               "dt_qk_norm_rope_table", rc)
    return qo, ko
  mode = _lib.ROPE_NONE
  pos_ptr = None
  dims = _lib.i32_array(0, 0, 0)
  theta = 1.0
  if rope is not None:
    if rope.mode not in _MODES:
      raise ValueError(f"rope mode {rope.mode!r}")
    mode = _MODES[rope.mode]
    pos = rope.positions
    if pos.shape != (s, 3):
      raise ValueError(f"positions must be ({s}, 3), got {tuple(pos.shape)}")
    pos = pos.to(device=dev, dtype=torch.int32).contiguous()
    pos_ptr = pos.data_ptr()
    dims = _lib.i32_array(*rope.axis_dims)
    theta = float(rope.theta)
  fn = lib.dt_qk_norm_rope_f32 if f32 else lib.dt_qk_norm_rope
  with torch.cuda.device(dev):
    rc = fn(
        q.data_ptr(), k.data_ptr(), qo.data_ptr(), ko.data_ptr(), b, s, h, d,
        _lib.strides3(q.stride()), _lib.strides3(ostr), wq.data_ptr(),
        wk.data_ptr(), float(eps), None if hs is None else hs.data_ptr(),
        mode, pos_ptr, dims, theta, vl, _lib.ptr(vl_dev), stream)
  _lib.check("dt_qk_norm_rope_f32" if f32 else "dt_qk_norm_rope", rc)
  return qo, ko
