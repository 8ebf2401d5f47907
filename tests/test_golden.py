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

from gpu_helpers import assert_prologue_close
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
    assert_prologue_close(got.float().cpu().numpy(), want, name)


# ---- table-driven RoPE, key smoothing and the fixed-m operand


def test_oracle_reproduces_table_and_smoothing_vectors(fx):
  from oracle import fixed_m as FM
  x, w = f32(fx["table_h3/x"]), fx["table_h3/w"]
  got = NR.h3_apply_rope_f64(NR.rms_norm_f64(x, w, 1e-5), fx["table_h3/cos"],
                             fx["table_h3/sin"])
  np.testing.assert_allclose(got, fx["table_h3/y"], atol=1e-6)
  x, w = f32(fx["table_moss/x"]), fx["table_moss/w"]
  got = NR.moss_rotate_f64(NR.rms_norm_f64(x, w, 1e-6), fx["table_moss/rows"])
  np.testing.assert_allclose(got, fx["table_moss/y"], atol=1e-6)
  ks, _ = FM.smooth_keys(f32(fx["ksmooth/k"]), int(fx["ksmooth/kv_len"][0]))
  np.testing.assert_array_equal(ks.astype(np.float32), fx["ksmooth/ks"])
  q, k = f32(fx["fixedm/q"]), f32(fx["fixedm/k"])
  mk = FM.fixed_m_operands(q * (1.44269504 / np.sqrt(128.0)),
                           np.repeat(k, 2, axis=1))
  np.testing.assert_array_equal(mk.astype(np.float32), fx["fixedm/mk"])


@pytest.mark.gpu
def test_gpu_table_smoothing_and_operand_vectors(fx):
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd as dta
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  from diffusers_tpu_amd.kernels.k_smoothing import smooth_keys
  g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
  bf = lambda name: g(f32(fx[name])).to(torch.bfloat16)
  # H3 tables
  x, w = bf("table_h3/x"), torch.from_numpy(fx["table_h3/w"])
  tab = dta.RopeTable.from_cos_sin(g(fx["table_h3/cos"]), g(fx["table_h3/sin"]))
  qo, _ = dta.qk_norm_rope(x, x, w, w, eps=1e-5, rope=tab, out_layout="bshd")
  torch.cuda.synchronize()
  assert_prologue_close(qo.float().cpu().numpy(), fx["table_h3/y"], "table_h3")
  # MOSS rows
  x, w = bf("table_moss/x"), torch.from_numpy(fx["table_moss/w"])
  tab = dta.RopeTable.from_sin_cos_rows(g(fx["table_moss/rows"]))
  qo, _ = dta.qk_norm_rope(x, x, w, w, rope=tab, out_layout="bshd")
  torch.cuda.synchronize()
  assert_prologue_close(qo.float().cpu().numpy(), fx["table_moss/y"],
                        "table_moss")
  # key smoothing: the mean's float32 sum may round to the other bf16
  # neighbour than the float64 one near a rounding boundary
  k = bf("ksmooth/k")
  ks = smooth_keys(k, int(fx["ksmooth/kv_len"][0]))
  torch.cuda.synchronize()
  want = fx["ksmooth/ks"]
  diff = np.abs(ks.float().cpu().numpy() - want)
  assert (diff <= 2.0 ** -6).all() and (diff == 0).mean() > 0.99
  # the fixed-m operand: flags equal, ceilings within one of each other
  q, k = bf("fixedm/q"), bf("fixedm/k")
  _, mk = fmb.fixed_m_prepare(q, k, smooth=False)
  torch.cuda.synchronize()
  got, want = mk.cpu().numpy(), fx["fixedm/mk"]
  np.testing.assert_array_equal(got[1], want[1])
  assert (np.abs(got[0] - want[0]) <= 1).all()
