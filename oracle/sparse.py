"""Block-sparse attention oracle (test infrastructure; see ``oracle/__init__.py``).

Restates the semantics of ``diffusers_tpu/kernels/sparse_splash.py``: query
rows of block ``i`` (``block_q`` rows, clamped to the sequence) see exactly
the keys of the key blocks listed for ``i`` (``block_kv`` keys each), below
``kv_len``; softmax over those keys only.  Also a set-based restatement of
the H3 temporal-window table (``models/minimax_h3/h3_tpu.py:213-224``).
"""
from __future__ import annotations

import math

import numpy as np


def window_table_bruteforce(seq, video_start, rows_per_frame, window, block_q,
                            block_kv):
  """Key block j is visited by query block i iff the query block starts in
  the text/audio prefix, or the key block does, or some query row r and key
  row c of the two blocks are at most ``window * rows_per_frame`` apart
  (explicit loops over rows and keys; small sizes only)."""
  reach = window * rows_per_frame
  nq, nk = -(-seq // block_q), -(-seq // block_kv)
  out = []
  for i in range(nq):
    rows = range(i * block_q, min((i + 1) * block_q, seq))
    keep = []
    for j in range(nk):
      cols = range(j * block_kv, min((j + 1) * block_kv, seq))
      near = any(abs(r - c) <= reach for r in rows for c in cols)
      if rows[0] < video_start or cols[0] < video_start or near:
        keep.append(j)
    out.append(keep)
  return out


def block_mask(sq, skv, block_q, block_kv, table):
  """Boolean ``[sq, skv]``: key c visible to query r under ``table``."""
  bq, bkv = min(block_q, sq), min(block_kv, skv)
  mask = np.zeros((sq, skv), bool)
  for i, row in enumerate(table):
    for j in row:
      mask[i * bq:(i + 1) * bq, j * bkv:(j + 1) * bkv] = True
  return mask


def attention_masked_f64(q, k, v, mask, *, scale=None):
  """float64 softmax attention over the keys ``mask`` allows.

  ``mask``: bool ``[Sq, Skv]`` shared by all heads or ``[Hq, Sq, Skv]``.
  Rows with no visible key come out as zeros.
  """
  q = np.asarray(q, np.float64)
  k = np.asarray(k, np.float64)
  v = np.asarray(v, np.float64)
  b, hq, sq, d = q.shape
  hkv = k.shape[1]
  scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
  mask = np.asarray(mask, bool)
  if mask.ndim == 2:
    mask = np.broadcast_to(mask, (hq,) + mask.shape)
  out = np.zeros((b, hq, sq, v.shape[-1]))
  for bi in range(b):
    for h in range(hq):
      kh = h // (hq // hkv)
      s = q[bi, h] @ k[bi, kh].T * scale
      s = np.where(mask[h], s, -np.inf)
      mx = s.max(axis=1, keepdims=True)
      live = np.isfinite(mx[:, 0])
      p = np.where(mask[h], np.exp(s - np.where(np.isfinite(mx), mx, 0)), 0)
      o = p @ v[bi, kh]
      o[live] /= p[live].sum(axis=1, keepdims=True)
      out[bi, h] = o
  return out
