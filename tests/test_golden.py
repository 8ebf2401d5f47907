"""Regression vectors (tests/golden/fixtures.npz, written by
tests/golden/make_fixtures.py from the float64 oracle).

CPU: the oracle still reproduces every stored output.  GPU: the HIP kernels,
called through the C ABI, match the stored outputs within the north-star
tolerances.
"""
import os

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import norm_rope as NR

PATH = os.path.join(os.path.dirname(__file__), "golden", "fixtures.npz")
ATTN = ["attn_d64", "attn_d128_gqa", "attn_d128_b2"]
ROPE = ["rope_half_3d", "rope_pair_qwen", "rope_half_1d_d64"]


@pytest.fixture(scope="module")
def fx():
  with np.load(PATH, allow_pickle=False) as z:
    return {k: z[k] for k in z.files}


def f32(bits):
  return (bits.astype(np.uint32) << 16).view(np.float32)


def _attn_meta(fx, name):
  kv_len, scale = fx[name + "/meta"]
  return (None if kv_len < 0 else int(kv_len)), (None if scale < 0 else float(scale))


def _rope_meta(fx, name):
  eps, vl, d0, d1, d2, mode = fx[name + "/meta"]
  return (float(eps), None if vl < 0 else int(vl), (int(d0), int(d1), int(d2)),
          "half" if mode == 0 else "pair")


@pytest.mark.parametrize("name", ATTN)
def test_oracle_reproduces_attention_vectors(fx, name):
  kv_len, scale = _attn_meta(fx, name)
  q, k, v = (f32(fx[name + "/" + t]) for t in "qkv")
  got = A.attention_f64(q, k, v, kv_len=kv_len, scale=scale)
  np.testing.assert_allclose(got, fx[name + "/o"], atol=1e-6)


@pytest.mark.parametrize("name", ROPE)
def test_oracle_reproduces_prologue_vectors(fx, name):
  eps, vl, dims, mode = _rope_meta(fx, name)
  got = NR.qk_norm_rope_f64(f32(fx[name + "/x"]), fx[name + "/w"], eps,
                            fx[name + "/pos"], dims, 1e4, mode, valid_len=vl)
  np.testing.assert_allclose(got, fx[name + "/y"], atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ATTN)
def test_gpu_attention_vectors(fx, name):
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd as dta
  kv_len, scale = _attn_meta(fx, name)
  q, k, v = (torch.from_numpy(f32(fx[name + "/" + t])).cuda().to(torch.bfloat16)
             for t in "qkv")
  out = dta.attention(q, k, v, scale=scale, block_q=0, block_kv=0,
                      block_kv_compute=0, kv_len=kv_len)
  torch.cuda.synchronize()
  err = np.abs(out.float().cpu().numpy() - fx[name + "/o"])
  assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())


@pytest.mark.gpu
@pytest.mark.parametrize("name", ROPE)
def test_gpu_prologue_vectors(fx, name):
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd as dta
  eps, vl, dims, mode = _rope_meta(fx, name)
  x = torch.from_numpy(f32(fx[name + "/x"])).cuda().to(torch.bfloat16)
  w = torch.from_numpy(fx[name + "/w"])
  rope = dta.RopeSpec(mode, torch.from_numpy(fx[name + "/pos"]).cuda(), dims, 1e4)
  qo, ko = dta.qk_norm_rope(x, x, w, w, eps=eps, rope=rope, valid_len=vl,
                            out_layout="bshd")
  torch.cuda.synchronize()
  want = fx[name + "/y"]
  for got in (qo, ko):
    err = np.abs(got.float().cpu().numpy() - want)
    assert (err <= 1e-2 + 2.0 ** -8 * np.abs(want)).all(), err.max()
