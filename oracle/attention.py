"""Dense attention oracle (test infrastructure; see ``oracle/__init__.py``).

Semantics follow the reference's normalized splash attention
(``diffusers_tpu/kernels/splash.py:566-650``): scores ``q.k * scale`` with
``scale = 1/sqrt(D)`` when ``None`` (``:607``); keys at or past ``kv_len``
masked (``:216-218``, masked score ``DEFAULT_MASK_VALUE`` ``:45`` whose
exp underflows to exactly 0, i.e. the same as ``-inf`` here); GQA maps query
head ``h`` to kv head ``h // (Hq // Hkv)`` (``:438-444``); output in query
layout ``[B, H, Sq, D]``.  Residual mode restates ``:665-742``: unnormalized
``o`` plus running max ``m`` and sum ``l`` in log2 units.
"""
from __future__ import annotations

import math

import numpy as np

LOG2_E = 1.44269504  # kernels/fixed_m_bound.py:37


def _kv_head_index(hq: int, hkv: int) -> np.ndarray:
  # kernels/splash.py:438-444: kv head = h // (Hq // Hkv)
  if hq % hkv:
    raise ValueError(f"{hq=} not a multiple of {hkv=}")
  return np.arange(hq) // (hq // hkv)


def attention_f64(q, k, v, *, scale=None, kv_len=None):
  """float64 dense softmax attention, [B,H,S,D] in/out.

  Follows kernels/splash.py:566-650 (normalized output) with the key mask of
  models/moss_image/jax_dit.py:183-187.  Row-chunked so large Skv fits.
  """
  q = np.asarray(q, np.float64)
  k = np.asarray(k, np.float64)
  v = np.asarray(v, np.float64)
  b, hq, sq, d = q.shape
  hkv, skv = k.shape[1], k.shape[2]
  scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
  n = skv if kv_len is None else int(kv_len)
  if not 1 <= n <= skv:
    raise ValueError(f"kv_len {n} outside [1, {skv}]")
  kvh = _kv_head_index(hq, hkv)
  out = np.empty((b, hq, sq, v.shape[-1]), np.float64)
  for bi in range(b):
    for h in range(hq):
      kk = k[bi, kvh[h], :n]
      vv = v[bi, kvh[h], :n]
      for s0 in range(0, sq, 1024):
        s = q[bi, h, s0:s0 + 1024] @ kk.T * scale
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[bi, h, s0:s0 + 1024] = (p @ vv) / p.sum(axis=1, keepdims=True)
  return out


def residual_f64(q, k, v, *, scale=None, kv_len=None):
  """Unnormalized (o, m, l) in log2 units, restating splash.py:665-742.

  m is the row max of ``q.k * scale * log2(e)`` and
  ``l = sum exp2(s - m)``, ``o = sum exp2(s - m) v`` (splash.py:250-267,
  emitted unnormalized at :362-367).  ``o / l`` equals ``attention_f64``.
  """
  q = np.asarray(q, np.float64)
  k = np.asarray(k, np.float64)
  v = np.asarray(v, np.float64)
  b, hq, sq, d = q.shape
  hkv, skv = k.shape[1], k.shape[2]
  scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
  n = skv if kv_len is None else int(kv_len)
  kvh = _kv_head_index(hq, hkv)
  o = np.empty((b, hq, sq, v.shape[-1]))
  m = np.empty((b, hq, sq, 1))
  l = np.empty((b, hq, sq, 1))
  for bi in range(b):
    for h in range(hq):
      s = q[bi, h] @ k[bi, kvh[h], :n].T * (scale * LOG2_E)
      mm = s.max(axis=1, keepdims=True)
      p = np.exp2(s - mm)
      m[bi, h], l[bi, h] = mm, p.sum(axis=1, keepdims=True)
      o[bi, h] = p @ v[bi, kvh[h], :n]
  return o, m, l


def attention_rows_f64(q, k, v, rows, *, scale=None, kv_len=None):
  """``attention_f64`` restricted to query rows ``rows`` (for huge Sq)."""
  q = np.asarray(q)[:, :, rows]
  return attention_f64(q, k, v, scale=scale, kv_len=kv_len)


def attention_torch_f32(q, k, v, *, scale=None, kv_len=None, threads=None):
  """torch-CPU float32 restatement (the CPU baseline leg).

  ``scaled_dot_product_attention`` with a boolean key mask — the same
  contract as the reference's CPU fallback ``jax.nn.dot_product_attention``
  with ``mask`` (models/moss_image/jax_dit.py:183-187).  Inputs are torch
  tensors on the CPU; output float32 [B,H,Sq,D].
  """
  import torch
  import torch.nn.functional as F
  if threads is not None:
    torch.set_num_threads(threads)
  q, k, v = (t.float() for t in (q, k, v))
  skv = k.shape[2]
  n = skv if kv_len is None else int(kv_len)
  if q.shape[1] != k.shape[1]:
    rep = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
  return F.scaled_dot_product_attention(q, k[:, :, :n], v[:, :, :n],
                                        scale=scale)
