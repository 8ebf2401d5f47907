"""Flash attention forward — drop-in for ``diffusers_tpu/kernels/splash.py``.

``attention`` keeps the reference's signature (kernels/splash.py:566-580) on
torch tensors ``[B, H, S, D]`` resident on the GPU, and runs the gfx950 HIP
kernels through the C ABI (``dt_flash_fwd_ex``: V row-major, or from
``PACKED_V_MIN_KEYS`` keys on in the packed layout of ``dt_pack_v``; a
workspace from torch's allocator lets the kernel split a partly filled last
round of workgroups over the keys).  ``residual_attention`` mirrors
kernels/splash.py:665-742 (unnormalized ``o`` plus ``m``, ``l`` in log2
units, for an LSE merge across KV shards).

Differences a caller can observe, all within the reference's tolerance:

* ``block_q``/``block_kv``/``block_kv_compute`` are TPU tile sizes; the
  gfx950 kernel has its own fixed tiling, so they are accepted and ignored
  (they only shaped the Pallas grid, kernels/splash.py:492-494;
  ``block_sizes`` resolves them to that tile and reports the launch plan).
* ``use_fixed_m`` runs the reference's fixed-m softmax (kernels/splash.py:
  170-248): the per-head bound comes from ``fixed_m_bound`` (one GPU pass over
  q and one over k), eligible heads start from the fixed reference ``m`` and
  the rest run online.  The normalized output is the same softmax either
  way; where the reference runs its last KV block online, this kernel
  re-bases only if a sum overflows.
* ``kv_mask_all`` picks between two masking schedules with identical output
  (kernels/splash.py:312-323); accepted and ignored.
* As in the reference (kernels/splash.py:607-609,633), ``q * scale *
  log2(e)`` is rounded to bf16 before the QK product (the kernel does this in
  registers with one rounding).
* Head dims: the kernels are built for 64, 128 and 256; any other multiple
  of 8 up to 256 runs zero-padded to the next of them (zero channels change
  no score; the extra output channels are dropped), with the scale of the
  real dim.  Above 256 (above 128 with ``qk_fp8``) raises
  ``NotImplementedError``, as does a dim that is not a multiple of 8
  (kernels/splash.py:156-160).
* ``qk_fp8`` casts K to E4M3 in one GPU pass (``fp8_cast``) and the kernel
  casts the scaled q to E4M3 in registers (kernels/splash.py:420-424); the
  QK product runs on the E4M3 MFMA, P and V stay bf16.
* Split query blocks (the tail split) round their probabilities to bf16
  against their own reference m, so a split and an unsplit run differ at
  bf16 rounding level; one shape always takes the same path.
"""
from __future__ import annotations

import functools
import math

import torch

from .. import _lib


def _check_bhsd(name, t):
  if not isinstance(t, torch.Tensor):
    raise TypeError(f"{name} must be a torch.Tensor")
  if t.dim() != 4:
    raise ValueError(f"{name} must be [B, H, S, D], got shape {tuple(t.shape)}")
  if not t.is_cuda:
    raise ValueError(f"{name} must be on the GPU (got {t.device}); the gfx950 "
                     "kernel has no CPU path")


def _check_same_device(device, **tensors):
  for name, t in tensors.items():
    if t.device != device:
      raise ValueError(f"{name} is on {t.device}, the query on {device}")


def _as_bf16_rows(t):
  """bf16 with a contiguous last axis and 8-aligned strides."""
  if t.dtype != torch.bfloat16:
    t = t.to(torch.bfloat16)
  if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or \
     t.data_ptr() % 16:
    t = t.contiguous()
  return t


class BlockSizes:
  """The reference's per-call tiling record (kernels/splash.py:92-112):
  ``block_q``, ``block_kv`` and ``block_kv_compute`` (default ``block_kv``).
  Kept so callers that build one keep working; the gfx950 kernel's own
  tile is fixed (``block_sizes.DEFAULT_BLOCKS``) and ``attention`` does not
  read these."""

  __slots__ = ("block_q", "block_kv", "block_kv_compute")

  def __init__(self, block_q, block_kv, block_kv_compute=None):
    self.block_q = block_q
    self.block_kv = block_kv
    self.block_kv_compute = (block_kv_compute if block_kv_compute is not None
                             else block_kv)


def kernel_head_dim(d, qk_fp8=False):
  """Head dim the gfx950 kernels run for a head dim ``d`` (a multiple of 8):
  64, 128 or 256; smaller dims are zero-padded up to it (zero channels add
  nothing to q.k and produce output channels that are dropped).  ``None``
  above 256, and above 128 with E4M3 keys."""
  if d > 256 or (qk_fp8 and d > 128):
    return None
  if d > 128:
    return 256
  if qk_fp8:
    return 128
  return 64 if d <= 64 else 128


def pad_head_dim(t, kd):
  """``t`` with its last axis zero-padded to ``kd`` (``t`` itself if equal)."""
  if t.shape[-1] == kd:
    return t
  return torch.nn.functional.pad(t, (0, kd - t.shape[-1]))


def _mk_operand(mk, hq, device):
  if not isinstance(mk, torch.Tensor) or mk.shape != (2, hq):
    raise ValueError(f"mk must be a (2, {hq}) tensor")
  return mk.to(device=device, dtype=torch.float32).contiguous()


class AttentionWorkspace:
  """Caller-owned scratch of ``attention`` / ``residual_attention``: the
  packed-V buffer (``dt_pack_v``) and the tail-split workspace
  (``dt_flash_fwd_ex``).

  Pass one instance to every call of a model (``workspace=ws``): the
  buffers are allocated on the first call that needs them and grow only when
  a later call needs more, so a 50-layer step allocates nothing after its
  first layer (at V7: 449 MB of packed V and 227 MiB of split workspace,
  which ``attention`` otherwise takes from torch's allocator per call).
  ``reserve`` sizes both up front, e.g. before capturing a HIP graph.
  Calls that share a workspace must be ordered on one stream; the contents
  do not outlive a call.
  """

  def __init__(self, device=None):
    self.device = torch.device("cuda" if device is None else device)
    if self.device.type == "cuda" and self.device.index is None:
      self.device = torch.device("cuda", torch.cuda.current_device())
    self._vt = None
    self._split = None
    self._views = {}

  def _get(self, attr, numel, dtype):
    buf = getattr(self, attr)
    if buf is None or buf.numel() < numel:
      buf = torch.empty(numel, device=self.device, dtype=dtype)
      setattr(self, attr, buf)
      self._views = {}
    view = self._views.get((attr, numel))
    if view is None:  # one view per size (slicing costs a microsecond)
      view = self._views[(attr, numel)] = buf[:numel]
    return view

  def packed_v(self, numel):
    """A bf16 buffer of at least ``numel`` elements for packed V."""
    return self._get("_vt", numel, torch.bfloat16)

  def split(self, nbytes):
    """A 16-byte aligned buffer of at least ``nbytes`` bytes for the split."""
    return self._get("_split", (nbytes + 3) // 4, torch.float32)

  def reserve(self, query_shape, key_shape, kv_len=None, *, packed=None):
    """Allocates what a call with these shapes needs (``kv_len`` an int or
    ``None``; a device length plans for every key).  ``packed``: whether
    the call streams packed V (default: as ``attention`` decides)."""
    b, hq, sq, d = query_shape
    _, hkv, skv, _ = key_shape
    # a device length, or per-sample lengths: plan for every key
    n = int(kv_len) if isinstance(kv_len, int) else skv
    if packed is None:
      packed = d == 128 and n >= PACKED_V_MIN_KEYS
    if packed:
      self.packed_v(packed_v_numel(b, hkv, n))
    with torch.cuda.device(self.device):
      nbytes = _lib.load().dt_flash_fwd_workspace_bytes(
          b, hq, sq, skv, 0 if n == skv else n, d)
    if nbytes:
      self.split(nbytes)
    return self


def _check_out(out, shape, device):
  if out is not None and (out.shape != shape or
                          out.dtype != torch.bfloat16 or
                          out.device != device or out.stride(-1) != 1 or
                          any(st % 4 for st in out.stride()[:3])):
    raise ValueError("out must be a bf16 [B, H, Sq, D] tensor on the "
                     "query's device with a contiguous last axis")


def _check_workspace(workspace, device):
  if workspace is None:
    return
  if not isinstance(workspace, AttentionWorkspace):
    raise TypeError("workspace must be an AttentionWorkspace")
  if workspace.device != device:
    raise ValueError(f"workspace is on {workspace.device}, the tensors on "
                     f"{device}")


def _launch(query, key, value, scale, kv_len, out=None, residual=False,
            mk=None, qk_fp8=False, packed_v=None, workspace=None):
  """One attention call through ``dt_flash_fwd_ex``.  ``packed_v``: V
  already packed by ``pack_v`` with the same kv_len (else V is packed here
  when the key count reaches ``PACKED_V_MIN_KEYS``, into ``workspace`` when
  given); ``workspace``: an ``AttentionWorkspace``."""
  for n, t in (("query", query), ("key", key), ("value", value)):
    _check_bhsd(n, t)
  _check_same_device(query.device, key=key, value=value)
  b, hq, sq, d = query.shape
  bk, hkv, skv, dk = key.shape
  if value.shape != key.shape:
    raise ValueError(f"value shape {tuple(value.shape)} != key shape "
                     f"{tuple(key.shape)}")
  if bk != b or dk != d:
    raise ValueError(f"query {tuple(query.shape)} / key {tuple(key.shape)} "
                     "disagree on batch or head dim")
  if d % 8:
    # kernels/splash.py:156-160 raises the same for head_dim_v % 8.
    raise NotImplementedError(f"head_dim={d} should be a multiple of 8")
  if hq % hkv:
    raise ValueError(f"{hq} query heads not a multiple of {hkv} kv heads")
  _check_workspace(workspace, query.device)
  n, n_dev = _lib.length_arg(kv_len, skv, query.device, batch=b)
  scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
  if not scale > 0:
    raise ValueError(f"scale must be positive, got {scale}")
  kd = kernel_head_dim(d, qk_fp8)
  if kd is None:
    raise NotImplementedError(f"head_dim={d}: the gfx950 kernels cover head "
                              "dims up to 256 (up to 128 with qk_fp8)")
  if not residual:
    _check_out(out, (b, hq, sq, d), query.device)
  if kd != d:
    if packed_v is not None:
      raise ValueError(f"packed_v is a head-dim-128 layout; head_dim={d} runs "
                       "zero-padded and packs its own V")
    # zero-padded channels: same scores, extra output channels dropped below
    res = _launch(pad_head_dim(query, kd), pad_head_dim(key, kd),
                  pad_head_dim(value, kd), scale,
                  n if n_dev is None else n_dev, residual=residual, mk=mk,
                  qk_fp8=qk_fp8, workspace=workspace)
    if residual:
      return res[0][..., :d].contiguous(), res[1], res[2]
    if out is not None:
      out.copy_(res[..., :d])
      return out
    return res[..., :d].contiguous()
  q = _as_bf16_rows(query)
  v = _as_bf16_rows(value)
  if qk_fp8:
    from .fp8_cast import quantize_saturating
    k = quantize_saturating(key)
  else:
    k = _as_bf16_rows(key)
  if mk is not None:
    mk = _mk_operand(mk, hq, q.device)
  mk_ptr = None if mk is None else mk.data_ptr()
  length = n if n_dev is None else n_dev
  if packed_v is None and d == 128 and (n_dev is not None or
                                        n >= PACKED_V_MIN_KEYS):
    # a device length plans for every key (the count is unknown here)
    if skv >= PACKED_V_MIN_KEYS:
      buf = None if workspace is None else \
          workspace.packed_v(packed_v_numel(b, hkv, skv if n_dev is not None
                                            else n))
      packed_v = pack_v(v, length, out=buf)
  return _call_ex(q, k, 1 if qk_fp8 else 0, v, packed_v, out, residual,
                  hkv, skv, scale, length, mk_ptr, workspace=workspace)


@functools.lru_cache(maxsize=4096)
def _split_bytes(b, hq, sq, skv, n, d, device_index):
  """``dt_flash_fwd_workspace_bytes`` per shape and device, queried once
  (the current device is ``device_index`` when it is called)."""
  return _lib.load().dt_flash_fwd_workspace_bytes(b, hq, sq, skv, n, d)


def _call_ex(q, k, k_format, v, packed_v, out, residual, hkv, skv, scale, n,
             mk_ptr, span=None, ids=None, workspace=None):
  """One ``dt_flash_fwd_ex`` call (``n``: int key length or a device int32
  tensor) with a tail-split workspace from ``workspace`` (an
  ``AttentionWorkspace``) or torch's allocator: returns ``o`` (``out`` if
  given) or ``(o32, m, l)``."""
  b, hq, sq, d = q.shape
  _check_workspace(workspace, q.device)
  lib = _lib.load()
  stream = torch.cuda.current_stream(q.device).cuda_stream
  s3 = lambda t: _lib.strides3(t.stride())
  n_dev = n if isinstance(n, torch.Tensor) else None
  # with a device length the host argument is its entry count
  n_host = _lib.dev_count(n_dev) if n_dev is not None else int(n)
  with torch.cuda.device(q.device):
    if residual:
      o = None
      o32 = torch.empty((b, hq, sq, d), device=q.device, dtype=torch.float32)
      m = torch.empty((b, hq, sq, 1), device=q.device, dtype=torch.float32)
      l = torch.empty((b, hq, sq, 1), device=q.device, dtype=torch.float32)
      outs = (None, None, o32.data_ptr(), m.data_ptr(), l.data_ptr())
    else:
      o = out if out is not None else torch.empty(
          (b, hq, sq, d), device=q.device, dtype=torch.bfloat16)
      outs = (o.data_ptr(), s3(o), None, None, None)
    nbytes = _split_bytes(b, hq, sq, skv, 0 if n_dev is not None else n_host,
                          d, q.device.index)
    if not nbytes:
      ws = None
    elif workspace is not None:
      ws = workspace.split(nbytes)
    else:
      ws = torch.empty((nbytes + 3) // 4, device=q.device, dtype=torch.float32)
    if packed_v is not None:
      vargs = (None, None, packed_v[0].data_ptr(), packed_v[1])
    else:
      vargs = (v.data_ptr(), s3(v), None, 0)
    rc = lib.dt_flash_fwd_ex(
        q.data_ptr(), k.data_ptr(), k_format, *vargs, outs[0], b, hq, hkv, sq,
        skv, d, s3(q), s3(k), outs[1], scale, n_host, _lib.ptr(n_dev), mk_ptr,
        None if span is None else span.data_ptr(),
        None if ids is None else ids.data_ptr(), *outs[2:],
        None if ws is None else ws.data_ptr(), nbytes, stream)
    _lib.check("dt_flash_fwd_ex", rc)
  if residual:
    return o32, m, l
  return o


# Key count from which the D = 128 path streams V from the packed layout
# (dt_pack_v).  The pass over V costs time linear in the keys, attention
# time quadratic: at ~6 TB/s against ~1.25 PFLOP/s the pass is about
# 208 / keys of the attention call, which the ~0.9 % it saves exceeds from
# about 23k keys on.
PACKED_V_MIN_KEYS = 32768


def packed_v_numel(b, hkv, n):
  """bf16 elements of the packed V of ``n`` keys (``pack_v``)."""
  return b * hkv * ((n + 63) // 64) * 64 * 128


def pack_v(value, kv_len=None, out=None):
  """``value`` ``(B, Hkv, S, 128)`` bf16 in the packed-V layout of
  ``dt_pack_v``: returns ``(vt, tiles)``, ``vt`` a flat bf16 tensor holding,
  per (batch, kv head), ``tiles`` contiguous ``[128][64]`` channel-major
  blocks of 64 keys (``out`` if given).  ``_launch(..., packed_v=(vt,
  tiles))`` takes it with the same ``kv_len`` (an int, or a device tensor:
  then every tile of the sequence is planned and the kernel skips those
  past the length it reads)."""
  b, hkv, skv, d = value.shape
  n, n_dev = _lib.length_arg(kv_len, skv, value.device, batch=b)
  tiles = ((skv if n_dev is not None else n) + 63) // 64
  size = b * hkv * tiles * 64 * 128
  if out is None:
    vt = torch.empty(size, device=value.device, dtype=torch.bfloat16)
  else:
    vt = out
    if (vt.dtype != torch.bfloat16 or vt.device != value.device or
        vt.numel() < size or not vt.is_contiguous()):
      raise ValueError(f"out must be a contiguous bf16 tensor of at least "
                       f"{size} elements on value's device")
  with torch.cuda.device(value.device):
    rc = _lib.load().dt_pack_v(
        value.data_ptr(), vt.data_ptr(), b, hkv, skv, d,
        _lib.i64_array(*value.stride()[:3]), n, _lib.ptr(n_dev), tiles,
        torch.cuda.current_stream(value.device).cuda_stream)
  _lib.check("dt_pack_v", rc)
  return vt, tiles


def attention(query, key, value, *, scale=None, block_q=None, block_kv=None,
              block_kv_compute=None, use_fixed_m=False, qk_fp8=False,
              kv_len=None, kv_mask_all=False, unroll=None, out=None,
              workspace=None):
  """Normalized non-causal attention (kernels/splash.py:566-650).

  Args:
    query: ``(B, heads, seq_q, dim)`` on the GPU, any float dtype.
    key: ``(B, kv_heads, seq_kv, dim)``; ``heads % kv_heads == 0`` (GQA,
      kernels/splash.py:438-444).
    value: same shape as ``key``.
    scale: softmax scale; ``None`` -> ``1/sqrt(dim)`` (:607).
    block_q, block_kv, block_kv_compute, unroll, kv_mask_all: accepted for
      signature compatibility (see module docstring).
    use_fixed_m: per-head fixed-m softmax, gated by
      ``fixed_m_bound.FIXED_M_SAFE_BOUND`` over this call's q and k; like the
      reference's gate it presumes k-smoothed keys (rowmax >= 0).
    qk_fp8: E4M3 Q/K into the QK product (kernels/splash.py:420-424); lossy,
      head_dim 128.
    kv_len: keys at or past it are masked: an int, or a one-element integer
      tensor.  A tensor on the GPU is read by the kernels when they run (the
      reference's traced scalar, :583-620): no host sync, and one captured
      HIP graph serves every length.  Per-sample lengths, one per batch
      element (the CFG pair of models/moss_image/jax_dit.py:181-210, which
      the reference runs as B calls), are a B-element GPU tensor or a host
      sequence of B ints: one launch, each batch element masked at its own
      length.  A device value <= 0 gives zero rows; one above seq_kv is
      clamped.  Padded keys should be zero, as the reference requires
      (:583-586).
    out: optional bf16 ``(B, heads, seq_q, dim)`` output (bf16 queries).
    workspace: optional ``AttentionWorkspace`` holding the packed-V buffer
      and the split workspace across calls (no per-call allocation).

  Returns:
    ``(B, heads, seq_q, dim)`` in ``query``'s dtype (``out`` if given).
  """
  del block_q, block_kv, block_kv_compute, unroll, kv_mask_all
  if out is not None and query.dtype != torch.bfloat16:
    raise ValueError("out= needs bf16 queries (the output has the query's "
                     "dtype)")
  return _attention(query, key, value, scale, use_fixed_m, qk_fp8, kv_len,
                    out=out, workspace=workspace)


def _attention(query, key, value, scale, use_fixed_m, qk_fp8, kv_len, *,
               k_norms=None, mk=None, out=None, workspace=None):
  """``attention``; ``k_norms``: the keys' per-head max row norms when the
  caller already has them (k_smoothing.smooth_keys), so the fixed-m bound
  reads only q; ``mk``: the whole fixed-m operand when the caller has it
  (fixed_m_bound.fixed_m_prepare)."""
  if use_fixed_m and mk is None:
    mk = _fixed_m_operand(query, key, scale, k_norms)
  if not use_fixed_m:
    mk = None
  res = _launch(query, key, value, scale, kv_len, mk=mk, qk_fp8=qk_fp8,
                out=out, workspace=workspace)
  return res if query.dtype == torch.bfloat16 else res.to(query.dtype)



def _fixed_m_operand(query, key, scale, k_norms=None):
  """kernels/splash.py:609-614: the (2, heads) operand over this call's
  q (scaled) and k, flat gate."""
  from . import fixed_m_bound as fmb
  _check_bhsd("query", query)
  _check_bhsd("key", key)
  if k_norms is None:  # q and k norms and the operand in one pipeline
    return fmb.fixed_m_prepare(query, key, scale, smooth=False,
                               gate=fmb.FIXED_M_SAFE_BOUND)[1]
  qn = fmb.fixed_m_query_norms(query, scale)
  kn = k_norms
  if kn.numel() != qn.numel():  # GQA: query head h reads kv head h // group
    kn = kn.repeat_interleave(qn.numel() // kn.numel())
  return fmb.fixed_m_operands_from_norms(qn, kn,
                                         gate=fmb.FIXED_M_SAFE_BOUND)


def residual_attention(query, key, value, *, scale=None, block_q=None,
                       block_kv=None, block_kv_compute=None, use_fixed_m=False,
                       qk_fp8=False, mk=None, kv_len=None, workspace=None):
  """Unnormalized ``(o, m, l)`` over one KV shard (kernels/splash.py:665-742).

  Returns ``o`` ``(B, heads, seq_q, dim)`` float32 (unnormalized, at scale
  ``2^-m``) and ``m``, ``l`` ``(B, heads, seq_q, 1)`` float32 with
  ``l = sum exp2(s - m)``, ``s = scale*log2(e)*q.k``.  ``m`` is the kernel's
  per-row scale reference, ``rowmax(s) - 13 < m <= rowmax(s)``, not always the
  max itself (the kernel moves it only when a tile's exp sum grows large).
  The reference's fixed-m residuals likewise carry a bound instead of the
  max, so shards are merged in LSE space (``m + log2(l)`` is exact), e.g. by
  ``merge_residuals``.

  With ``use_fixed_m`` the ``(2, heads)`` operand ``mk`` is required
  (kernels/splash.py:712-713), e.g. ``fixed_m_bound.ring_fixed_m_operands``;
  a fixed head's ``m`` is then ``mk[0, h] - 88`` (raised only if a sum
  overflows), a bound rather than the row max.
  ``kv_len`` and ``workspace`` as in ``attention``.

  Raises:
    ValueError: ``use_fixed_m`` without ``mk``.
  """
  del block_q, block_kv, block_kv_compute
  if use_fixed_m and mk is None:
    raise ValueError("use_fixed_m needs the (2, heads) operand mk.")
  return _launch(query, key, value, scale, kv_len, residual=True,
                 mk=mk if use_fixed_m else None, qk_fp8=qk_fp8,
                 workspace=workspace)


def merge_residuals(parts):
  """LSE-space merge of residual ``(o, m, l)`` triples from KV shards.

  The merge an outer ring loop performs (kernels/splash.py:653-664): m is a
  common scale, so ``o = sum 2^(m_i - M) o_i``, ``l = sum 2^(m_i - M) l_i``
  with ``M = max m_i``; the normalized output is ``o / l``.
  """
  ms = torch.stack([p[1] for p in parts])
  big = ms.max(dim=0).values
  o = sum(torch.exp2(p[1] - big) * p[0] for p in parts)
  l = sum(torch.exp2(p[1] - big) * p[2] for p in parts)
  return o / l
