"""ctypes binding of libdt_attention.so (the C ABI in include/dt_attention.h).

This module is the only place that touches the shared library.  There is no
CPU or eager fallback: if the library is missing or a call fails, an
exception is raised.
"""
from __future__ import annotations

import ctypes
import functools
import threading
from pathlib import Path

from . import _build

DT_OK = 0
DT_ERR_ARG = -1
DT_ERR_SHAPE = -2
DT_ERR_UNSUPPORTED = -3
DT_ERR_LAUNCH = -4

ROPE_NONE, ROPE_HALF, ROPE_PAIR = 0, 1, 2

# static scratch of dt_flash_fwd_ex_noalloc (DT_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 64 << 20

# Every symbol the header declares, with its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_L = ctypes.c_int64
_Z = ctypes.c_size_t
SIGNATURES = {
    "dt_version": (_I, []),
    "dt_last_error": (ctypes.c_char_p, []),
    "dt_qk_norm_rope": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P,
                             _F, _P, _I, _P, _P, _F, _I, _P, _P]),
    "dt_qk_norm_rope_f32": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P,
                                 _P, _F, _P, _I, _P, _P, _F, _I, _P, _P]),
    "dt_qk_norm_rope_table": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P,
                                   _P, _P, _F, _P, _I, _P, _P, _P, _I, _I,
                                   _P, _P]),
    "dt_qk_norm_rope_table_f32": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P,
                                       _P, _P, _P, _F, _P, _I, _P, _P, _P,
                                       _I, _I, _P, _P]),
    "dt_flash_fwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P,
                          _P, _F, _I, _P, _P, _P, _P, _P]),
    "dt_max_row_norm": (_I, [_P, _I, _I, _I, _I, _P, _F, _P, _P]),
    "dt_flash_fwd_qk8": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P,
                              _P, _P, _F, _I, _P, _P, _P, _P, _P]),
    "dt_quantize_e4m3": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _F, _P]),
    "dt_flash_fwd_blocksparse": (_I, [_P, _P, _I, _P, _P, _I, _I, _I, _I, _I,
                                      _I, _P, _P, _P, _P, _F, _I, _P, _P, _P,
                                      _P, _P, _P, _P]),
    "dt_pack_v": (_I, [_P, _P, _I, _I, _I, _I, _P, _I, _P, _L, _P]),
    "dt_flash_fwd_ex": (_I, [_P, _P, _I, _P, _P, _P, _L, _P, _I, _I, _I, _I,
                             _I, _I, _P, _P, _P, _F, _I, _P, _P, _P, _P, _P,
                             _P, _P, _P, _Z, _P]),
    "dt_flash_fwd_workspace_bytes": (_Z, [_I, _I, _I, _I, _I, _I]),
    "dt_flash_fwd_plan": (_I, [_I, _I, _I, _I, _I, _I, _Z, _P, _P]),
    "dt_flash_fwd_ex_noalloc": (_I, [_P, _P, _I, _P, _P, _P, _L, _P, _I, _I,
                                     _I, _I, _I, _I, _P, _P, _P, _F, _I, _P,
                                     _P, _P, _P, _P, _P, _P, _Z, _P]),
    "dt_smooth_keys": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P,
                            _Z, _P]),
    "dt_smooth_keys_workspace_bytes": (_Z, [_I, _I, _I, _I, _I]),
    "dt_fixed_m_prepare": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P,
                                _P, _I, _P, _F, _F, _I, _P, _P, _Z, _P]),
    "dt_fixed_m_prepare_workspace_bytes": (_Z, [_I] * 8),
}

_lock = threading.Lock()
_lib = None


class DtError(RuntimeError):
  """A non-zero status from the C ABI."""

  def __init__(self, fn: str, code: int, msg: str):
    super().__init__(f"{fn} failed ({code}): {msg}")
    self.code = code


def load(path: Path | None = None) -> ctypes.CDLL:
  """Loads (once) and returns the library; raises if it is not built."""
  global _lib
  with _lock:
    if _lib is not None and path is None:
      return _lib
    p = Path(path) if path is not None else _build.LIB_PATH
    if not p.exists():
      raise RuntimeError(
          f"{p} is not built; run `python -c 'import __graft_entry__ as g; "
          "g.build()'` (or python -m diffusers_tpu_amd._build)")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
      fn = getattr(lib, name)
      fn.restype = res
      fn.argtypes = args
    if path is None:
      _lib = lib
    return lib


def check(fn: str, code: int) -> None:
  if code != DT_OK:
    msg = load().dt_last_error().decode(errors="replace")
    if code in (DT_ERR_ARG, DT_ERR_SHAPE):
      raise ValueError(f"{fn}: {msg}")
    if code == DT_ERR_UNSUPPORTED:
      raise NotImplementedError(f"{fn}: {msg}")
    raise DtError(fn, code, msg)


def i64_array(*vals) -> ctypes.Array:
  return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


@functools.lru_cache(maxsize=1024)
def strides3(strides: tuple) -> ctypes.Array:
  """The (b, h, s) element strides of a tensor as the C ABI takes them,
  one shared read-only array per distinct tuple (building a ctypes array
  costs about a microsecond, a visible share of a small call)."""
  return i64_array(*strides[:3])


_host_lengths = {}


def length_arg(n, limit, device, name="kv_len", batch=None):
  """A length argument of the C ABI as ``(host_int, device_tensor)``.

  ``None`` -> ``(limit, None)``; a Python int (or a one-element CPU tensor,
  read on the host) -> ``(n, None)`` after a range check; a one-element
  tensor on the GPU -> ``(0, int32 tensor)``: the kernels read it when they
  run (the reference's traced kv_len scalar, kernels/splash.py:583-620),
  with no host synchronization, so one captured HIP graph serves every
  length.

  Per-sample lengths (``batch`` = B > 1): a ``B``-element GPU tensor ->
  ``(B, int32 tensor)``, entry b for batch element b (the MOSS CFG pair's
  ``kv_len[B]``, models/moss_image/jax_dit.py:181-210); a host sequence or
  CPU tensor of B ints -> range checked, then ``(n, None)`` when all are
  equal, else ``(B, int32 tensor)`` on ``device`` (one cached copy per
  distinct tuple).  With a device tensor the host int is the entry count
  the C ABI takes beside the pointer.

  A device value <= 0 means no keys (the empty result) and one above
  ``limit`` means ``limit``; neither can be range checked on the host.
  Keep the returned tensor alive until the call is enqueued.
  """
  import torch
  if n is None:
    return limit, None
  per_sample = batch is not None and batch > 1
  if isinstance(n, torch.Tensor):
    if n.is_floating_point() or n.is_complex() or n.dtype == torch.bool:
      raise ValueError(f"{name} must be an integer tensor")
    if n.numel() != 1 and not (per_sample and n.numel() == batch):
      want = f"a scalar or {batch} per-sample values" if per_sample else \
          "a scalar"
      raise ValueError(f"{name} must be {want}, got {n.numel()} values")
    if n.is_cuda:
      if device is not None and n.device != device:
        raise ValueError(f"{name} is on {n.device}, the call runs on {device}")
      t = n.reshape(-1)
      if t.dtype != torch.int32:
        t = t.to(torch.int32)
      return (0 if t.numel() == 1 else t.numel()), t.contiguous()
    n = n.reshape(-1).tolist()
    if len(n) == 1:
      n = n[0]
  if not isinstance(n, (int, str)) and hasattr(n, "__len__"):
    vals = [int(x) for x in n]  # a list, tuple or NumPy array of ints
    if len(vals) == 1:
      n = vals[0]
    else:
      if not per_sample or len(vals) != batch:
        raise ValueError(f"{name} has {len(vals)} values for batch {batch}")
      for x in vals:
        if not 1 <= x <= limit:
          raise ValueError(f"{name}={x} outside [1, {limit}]")
      if len(set(vals)) == 1:
        return vals[0], None
      if device is None:
        raise ValueError(f"per-sample {name} needs a device")
      key = (tuple(vals), str(device))
      t = _host_lengths.get(key)
      if t is None:
        if len(_host_lengths) > 256:
          _host_lengths.clear()
        t = _host_lengths[key] = torch.tensor(vals, dtype=torch.int32,
                                              device=device)
      return len(vals), t
  n = int(n)
  if not 1 <= n <= limit:
    raise ValueError(f"{name}={n} outside [1, {limit}]")
  return n, None


def dev_count(t) -> int:
  """The entry count the C ABI takes beside a device length tensor."""
  return 0 if t is None or t.numel() == 1 else t.numel()


def ptr(t):
  """Device pointer of a tensor, or None."""
  return None if t is None else t.data_ptr()


def i32_array(*vals) -> ctypes.Array:
  return (ctypes.c_int32 * len(vals))(*[int(v) for v in vals])
