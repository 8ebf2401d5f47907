"""Block-sparse flash attention — mirror of ``diffusers_tpu/kernels/sparse_splash.py``.

Same arithmetic as ``splash.attention``; the key sweep of each query block
walks a table of key blocks instead of every block, so skipped blocks cost
neither memory traffic nor MFMA work (kernels/sparse_splash.py:1-5).  A
full table reproduces the dense kernel exactly.

The reference's tables are in its own ``(block_q, block_kv)`` units: per
query block, the sorted key blocks it visits, shared by all heads, or
``(classes, head_class)`` with one table per head class
(kernels/sparse_splash.py:439-462).  The gfx950 kernel works in 256-row
query blocks and 64-key tiles (``DT_SPARSE_Q_BLOCK``/``DT_SPARSE_KV_TILE``),
so a table converts exactly when ``block_q`` is a multiple of 256 and
``block_kv`` of 64 (after clamping to the sequence lengths, as
``_local_blocks`` does, :537-565); other block sizes raise
``NotImplementedError``.  ``TileTable`` holds a converted table on the GPU
so repeated calls skip the conversion.

``temporal_window_table`` restates the H3 temporal-window table
(models/minimax_h3/h3_tpu.py:213-224).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from .. import _lib
from . import splash

Q_BLOCK = 256   # DT_SPARSE_Q_BLOCK
KV_TILE = 64    # DT_SPARSE_KV_TILE

BlockSizes = splash.BlockSizes  # kernels/sparse_splash.py:87 has its own copy


def temporal_window_table(seq, video_start, rows_per_frame, window, block_q,
                          block_kv):
  """Each query block's key blocks, ascending (h3_tpu.py:213-224).

  Query blocks that start before ``video_start`` (text/audio rows) attend to
  everything; key blocks that start before it are always kept; otherwise a
  key block is kept when it overlaps the query block widened by
  ``window * rows_per_frame`` rows on each side.
  """
  reach = window * rows_per_frame
  num_q, num_kv = -(-seq // block_q), -(-seq // block_kv)
  rows = []
  for i in range(num_q):
    q0, q1 = i * block_q, min((i + 1) * block_q, seq)
    rows.append([
        j for j in range(num_kv)
        if q0 < video_start or j * block_kv < video_start
        or (j * block_kv < q1 + reach
            and min((j + 1) * block_kv, seq) > q0 - reach)])
  return rows


@dataclass
class TileTable:
  """A block-sparse table in kernel units, resident on the GPU.

  ``span``: int32 ``(heads, ceil(Sq/256), 2)`` begin/end into ``ids``;
  ``ids``: int32 64-key tile indices.  ``sq``, ``kv_len`` record what it was
  built for.
  """
  span: torch.Tensor
  ids: torch.Tensor
  sq: int
  kv_len: int
  kept_tiles: int
  full_tiles: int


def _classes(kv_table, hq):
  if isinstance(kv_table, tuple):
    classes, head_class = kv_table
    head_class = [int(c) for c in head_class]
    if len(head_class) != hq:
      raise ValueError(f"head_class has {len(head_class)} entries, need {hq}")
    return [list(t) for t in classes], head_class
  return [list(kv_table)], [0] * hq


def build_tile_table(kv_table, *, sq, skv, heads, block_q, block_kv,
                     kv_len=None, device="cuda"):
  """Converts a reference-format table to a ``TileTable``.

  ``kv_table`` is a list (per query block of ``block_q`` rows) of key-block
  indices (``block_kv`` keys each), or ``(classes, head_class)``.  Block
  sizes are clamped to the sequence lengths first (sparse_splash.py:537-565).
  Key tiles at or past ``kv_len`` are dropped.
  """
  bq, bkv = min(int(block_q), sq), min(int(block_kv), skv)
  if bq % Q_BLOCK and bq != sq:
    raise NotImplementedError(
        f"block_q={block_q}: the gfx950 kernel's 256-row query blocks must "
        "each fall inside one table row (block_q a multiple of 256)")
  if bkv % KV_TILE and bkv != skv:
    raise NotImplementedError(
        f"block_kv={block_kv}: table key blocks must be whole 64-key tiles "
        "(block_kv a multiple of 64)")
  n = int(kv_len) if kv_len is not None else skv
  if not 1 <= n <= skv:
    raise ValueError(f"kv_len={n} outside [1, {skv}]")
  n_tiles_valid = -(-n // KV_TILE)
  n_tiles_all = -(-skv // KV_TILE)
  num_q, num_kv = -(-sq // bq), -(-skv // bkv)
  nqb = -(-sq // Q_BLOCK)
  classes, head_class = _classes(kv_table, heads)
  # per class: tile list of each kernel query block
  class_rows = []
  for t in classes:
    if len(t) != num_q:
      raise ValueError(f"table has {len(t)} rows, need {num_q} "
                       f"(seq_q={sq}, block_q={bq})")
    rows = []
    for r in t:
      r = [int(j) for j in r]
      if any(j < 0 or j >= num_kv for j in r):
        raise ValueError(f"key block out of range [0, {num_kv}) in {r}")
      if len(set(r)) != len(r):
        raise ValueError(f"repeated key block in {r}")
      tiles = []
      for j in sorted(r):
        t0 = j * bkv // KV_TILE
        t1 = min(-(-min((j + 1) * bkv, skv) // KV_TILE), n_tiles_all)
        tiles.extend(range(t0, min(t1, n_tiles_valid)))
      if not tiles:
        raise ValueError("a table row visits no key below kv_len")
      rows.append(tiles)
    class_rows.append([rows[i * Q_BLOCK // bq] for i in range(nqb)])
  ids, offsets = [], []
  for rows in class_rows:
    off = []
    for tiles in rows:
      off.append((len(ids), len(ids) + len(tiles)))
      ids.extend(tiles)
    offsets.append(off)
  span = np.array([offsets[c] for c in head_class], np.int32)
  kept = sum(e - b for c in head_class for b, e in offsets[c])
  return TileTable(
      span=torch.from_numpy(span).to(device),
      ids=torch.from_numpy(np.asarray(ids, np.int32)).to(device),
      sq=sq, kv_len=n, kept_tiles=kept,
      full_tiles=heads * nqb * n_tiles_valid)


def _dyn_table(kv_table_dyn):
  """``(table, counts)`` arrays (sparse_splash.py:441-444): rows padded to a
  common width; counts says how many entries of each row are real."""
  table, counts = kv_table_dyn
  table = np.asarray(table.cpu() if torch.is_tensor(table) else table)
  counts = np.asarray(counts.cpu() if torch.is_tensor(counts) else counts)
  if table.ndim == 2:
    table, counts = table[None], counts.reshape(1, -1)
  # the reference reads class 0 for every head on this path (:441-444)
  return [list(table[0, i, :int(counts[0, i])]) for i in range(table.shape[1])]


def _launch_sparse(query, key, value, scale, kv_len, table, *, residual,
                   mk=None, qk_fp8=False):
  for nm, t in (("query", query), ("key", key), ("value", value)):
    splash._check_bhsd(nm, t)
  splash._check_same_device(query.device, key=key, value=value)
  b, hq, sq, d = query.shape
  _, hkv, skv, _ = key.shape
  if value.shape != key.shape or key.shape[0] != b or key.shape[-1] != d:
    raise ValueError("query/key/value shapes disagree")
  if d % 8 or d > 128:
    raise NotImplementedError(f"head_dim={d}: block-sparse attention covers "
                              "multiples of 8 up to 128")
  if d != 128:
    # zero-padded channels: same scores; the extra output channels dropped
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    res = _launch_sparse(*(splash.pad_head_dim(t, 128)
                           for t in (query, key, value)),
                         scale, kv_len, table, residual=residual, mk=mk,
                         qk_fp8=qk_fp8)
    if residual:
      return res[0][..., :d].contiguous(), res[1], res[2]
    return res[..., :d].contiguous()
  if hq % hkv:
    raise ValueError(f"{hq} query heads not a multiple of {hkv} kv heads")
  n = _host_kv_len(kv_len, skv)
  if table.sq != sq or table.kv_len != n or table.span.shape[0] != hq:
    raise ValueError("TileTable was built for another shape or kv_len")
  scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
  q = splash._as_bf16_rows(query)
  v = splash._as_bf16_rows(value)
  if qk_fp8:
    from .fp8_cast import quantize_saturating
    k, k_format = quantize_saturating(key), 1
  else:
    k, k_format = splash._as_bf16_rows(key), 0
  if mk is not None:
    mk = splash._mk_operand(mk, hq, q.device)
  mk_ptr = None if mk is None else mk.data_ptr()
  span = table.span.to(q.device).contiguous()
  ids = table.ids.to(q.device).contiguous()
  # packed V pays when the visited share of the attention work still
  # outweighs the pass over all of V (splash.PACKED_V_MIN_KEYS at full
  # density)
  packed = None
  if n * table.kept_tiles >= splash.PACKED_V_MIN_KEYS * table.full_tiles:
    packed = splash.pack_v(v, n)
  return splash._call_ex(q, k, k_format, v, packed, None, residual, hkv, skv,
                         scale, n, mk_ptr, span, ids)


def _host_kv_len(kv_len, skv):
  """The key length as a host int: the tile table lists the tiles below it,
  so block-sparse calls take no device-side length."""
  if isinstance(kv_len, torch.Tensor) and kv_len.is_cuda:
    raise ValueError("block-sparse attention builds its tile table on the "
                     "host: pass kv_len as an int (or a CPU tensor)")
  return _lib.length_arg(kv_len, skv, None)[0]


def _table_for(query, key, block_q, block_kv, kv_table, kv_table_dyn, kv_len):
  if isinstance(kv_table, TileTable):
    return kv_table
  sq, skv, hq = query.shape[2], key.shape[2], query.shape[1]
  if kv_table_dyn is not None:
    kv_table = _dyn_table(kv_table_dyn)
  if kv_table is None:
    bkv = min(int(block_kv), skv)
    nq = -(-sq // min(int(block_q), sq))
    kv_table = [list(range(-(-skv // bkv)))] * nq
  n = _host_kv_len(kv_len, skv)
  return build_tile_table(kv_table, sq=sq, skv=skv, heads=hq, block_q=block_q,
                          block_kv=block_kv, kv_len=n, device=query.device)


def attention(query, key, value, *, scale=None, block_q, block_kv,
              block_kv_compute=None, use_fixed_m=False, qk_fp8=False,
              kv_table=None, kv_table_dyn=None, kv_len=None):
  """Normalized block-sparse attention (kernels/sparse_splash.py:568-662).

  ``kv_table``: per query block (``block_q`` rows) the sorted key blocks
  (``block_kv`` keys) to visit, or ``(classes, head_class)``, or a
  ``TileTable``; ``None`` visits every block.  ``kv_table_dyn``:
  ``(table, counts)`` arrays instead.  Other arguments as
  ``splash.attention``.
  """
  del block_kv_compute
  table = _table_for(query, key, block_q, block_kv, kv_table, kv_table_dyn,
                     kv_len)
  mk = splash._fixed_m_operand(query, key, scale) if use_fixed_m else None
  out = _launch_sparse(query, key, value, scale, kv_len, table,
                       residual=False, mk=mk, qk_fp8=qk_fp8)
  return out if query.dtype == torch.bfloat16 else out.to(query.dtype)


def residual_attention(query, key, value, *, scale=None, block_q, block_kv,
                       block_kv_compute=None, use_fixed_m=False, qk_fp8=False,
                       mk=None, kv_table=None, kv_table_dyn=None,
                       kv_len=None):
  """Unnormalized ``(o, m, l)`` (kernels/sparse_splash.py:664-741).

  The reference's residual form visits every key block; ``kv_table`` /
  ``kv_len`` are accepted here as well.  ``mk`` is required with
  ``use_fixed_m``.
  """
  del block_kv_compute
  if use_fixed_m and mk is None:
    raise ValueError("use_fixed_m needs the (2, heads) operand mk.")
  table = _table_for(query, key, block_q, block_kv, kv_table, kv_table_dyn,
                     kv_len)
  return _launch_sparse(query, key, value, scale, kv_len, table,
                        residual=True, mk=mk if use_fixed_m else None,
                        qk_fp8=qk_fp8)
