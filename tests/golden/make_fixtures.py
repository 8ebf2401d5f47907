"""Writes tests/golden/fixtures.npz: small seeded cases with float64 oracle
outputs (oracle/), used as regression vectors for the oracle and the GPU
kernels.  The reference path cannot run in this environment (JAX/Pallas,
Python >= 3.12, no network), so the expected outputs come from the oracle,
which tests/test_oracle.py pins against library routines, brute force and
closed forms.

Inputs are rounded to bf16 and stored as bf16 bit patterns (uint16), so the
GPU kernels see exactly the oracle's inputs; outputs are float32.

    python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as A  # noqa: E402
from oracle import fixed_m as FM  # noqa: E402
from oracle import norm_rope as NR  # noqa: E402


def bf16(x):
  """bf16-rounded values, returned as float32."""
  return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def bits(x):
  """bf16 bit patterns (uint16) of bf16-exact float32 values."""
  return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def main():
  rng = np.random.default_rng(20261201)
  out = {}
  # attention: (name, B, Hq, Hkv, Sq, Skv, D, kv_len, scale)
  cases = [("attn_d64", 1, 2, 2, 64, 100, 64, 90, None),
           ("attn_d128_gqa", 1, 4, 2, 40, 130, 128, 101, 0.1),
           ("attn_d128_b2", 2, 1, 1, 33, 64, 128, None, None)]
  for name, b, hq, hkv, sq, skv, d, kv_len, scale in cases:
    q = bf16(rng.standard_normal((b, hq, sq, d)))
    k = bf16(rng.standard_normal((b, hkv, skv, d)))
    v = bf16(rng.standard_normal((b, hkv, skv, d)))
    o = A.attention_f64(q, k, v, kv_len=kv_len, scale=scale)
    out[name + "/q"], out[name + "/k"], out[name + "/v"] = bits(q), bits(k), bits(v)
    out[name + "/o"] = o.astype(np.float32)
    out[name + "/meta"] = np.array([-1 if kv_len is None else kv_len,
                                    -1.0 if scale is None else scale])
  # prologue: (name, B, S, H, D, mode, axis_dims, eps, valid_len)
  pcases = [("rope_half_3d", 1, 20, 3, 128, "half", (44, 42, 42), 1e-6, None),
            ("rope_pair_qwen", 1, 17, 2, 128, "pair", (16, 56, 56), 1e-6, 15),
            ("rope_half_1d_d64", 2, 9, 2, 64, "half", (64, 0, 0), 1e-5, None)]
  for name, b, s, h, d, mode, dims, eps, vl in pcases:
    x = bf16(rng.standard_normal((b, s, h, d)))
    w = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    pos = rng.integers(0, 90, size=(s, 3)).astype(np.int32)
    y = NR.qk_norm_rope_f64(x, w, eps, pos, dims, 1e4, mode, valid_len=vl)
    out[name + "/x"], out[name + "/w"], out[name + "/pos"] = bits(x), w, pos
    out[name + "/y"] = y.astype(np.float32)
    out[name + "/meta"] = np.array([eps, -1 if vl is None else vl, *dims,
                                    0 if mode == "half" else 1], np.float64)
  # table-driven RoPE (appended after the cases above, so their values do
  # not move): H3's apply_rope with (S, rotary) tables of repeated halves,
  # MOSS's _rotate with per-batch (B, S, D) [sin | cos] rows
  x = bf16(rng.standard_normal((1, 11, 2, 128)))
  w = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
  ang = rng.uniform(0, 40, size=(11, 48))
  cos = np.cos(np.concatenate([ang, ang], -1)).astype(np.float32)
  sin = np.sin(np.concatenate([ang, ang], -1)).astype(np.float32)
  y = NR.h3_apply_rope_f64(NR.rms_norm_f64(x, w, 1e-5), cos, sin)
  out.update({"table_h3/x": bits(x), "table_h3/w": w, "table_h3/cos": cos,
              "table_h3/sin": sin, "table_h3/y": y.astype(np.float32)})
  x = bf16(rng.standard_normal((2, 9, 2, 128)))
  w = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
  ang = rng.uniform(0, 40, size=(2, 9, 64))
  rows = np.concatenate([np.sin(ang), np.cos(ang)], -1).astype(np.float32)
  y = NR.moss_rotate_f64(NR.rms_norm_f64(x, w, 1e-6), rows)
  out.update({"table_moss/x": bits(x), "table_moss/w": w,
              "table_moss/rows": rows, "table_moss/y": y.astype(np.float32)})
  # key smoothing with padded rows (jax_server.py:271-289)
  k = bf16(rng.standard_normal((2, 3, 50, 64)) + 2.0)
  ks, _ = FM.smooth_keys(k, kv_len=41)
  out.update({"ksmooth/k": bits(k), "ksmooth/ks": ks.astype(np.float32),
              "ksmooth/kv_len": np.array([41])})
  # the fixed-m operand (fixed_m_bound.py:98-118), GQA 4 query heads on 2
  q = bf16(rng.standard_normal((1, 4, 40, 128)))
  q[:, 3] *= 12
  q = bf16(q)
  k = bf16(rng.standard_normal((1, 2, 60, 128)))
  c = 1.44269504 / np.sqrt(128.0)
  kr = np.repeat(k, 2, axis=1)
  mk = FM.fixed_m_operands(q.astype(np.float64) * c, kr)
  out.update({"fixedm/q": bits(q), "fixedm/k": bits(k),
              "fixedm/mk": mk.astype(np.float32)})
  path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.npz")
  np.savez_compressed(path, **out)
  print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
  main()
