"""Key smoothing on the GPU (dt_smooth_keys, kernels/k_smoothing.py) against
the oracle's restatement of models/minimax_h3/jax_server.py:271-289."""
import numpy as np
import pytest
import torch

from gpu_helpers import banner, seeded, to64
from oracle import fixed_m as FM

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ksm():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.kernels import k_smoothing
  return k_smoothing


def _check(got, k, kv_len):
  want, mean = FM.smooth_keys(to64(k), kv_len)
  g = to64(got)
  diff = np.abs(g - want)
  # the kernel's float32 mean and the oracle's float64 one round to the same
  # bf16 except within float32 error of a rounding boundary: there the
  # result may move by one bf16 step of the mean
  tol = 2.0 ** -8 * (np.abs(mean) + np.abs(want)) + 1e-30
  assert (diff <= tol).all(), float(diff.max())
  assert (diff == 0).mean() > 0.999


@pytest.mark.parametrize("shape,kv_len", [
    ((2, 3, 1000, 128), None),
    ((1, 4, 777, 128), 701),       # padded rows
    ((1, 2, 300, 64), None),
    ((2, 2, 5000, 64), 4321),
])
def test_smooth_matches_oracle(ksm, shape, kv_len):
  banner(f"smooth_keys {shape} kv_len={kv_len}")
  k = seeded(shape, 190) + 1.5        # a mean worth removing
  ks, kn = ksm.smooth_keys(k, kv_len, norms=True)
  torch.cuda.synchronize()
  _check(ks, k, kv_len)
  want = FM.max_row_norm_per_head(to64(ks))
  np.testing.assert_allclose(to64(kn), want, rtol=2e-6)
  if kv_len is not None:
    assert torch.all(ks[:, :, kv_len:] == 0)


def test_smooth_strided_inplace_deterministic(ksm):
  banner("smooth_keys strided / in place / repeat")
  base = seeded((1, 600, 4, 128), 191) - 0.7
  k = base.transpose(1, 2)              # (B, H, S, D) view of BSHD storage
  a = ksm.smooth_keys(k)
  b = ksm.smooth_keys(k.contiguous())
  c = ksm.smooth_keys(k)
  kk = k.contiguous()
  ksm.smooth_keys(kk, out=kk)
  torch.cuda.synchronize()
  assert torch.equal(a, b) and torch.equal(a, c) and torch.equal(a, kk)
  _check(a, k, None)


def test_smooth_other_head_dims_use_torch(ksm):
  banner("smooth_keys D=96 (torch ops)")
  k = seeded((1, 2, 200, 96), 192) + 1.0
  ks = ksm.smooth_keys(k, 150)
  torch.cuda.synchronize()
  _check(ks, k, 150)


def test_fixed_m_dispatch_uses_fused_bound():
  """The dispatch's fixed-m op smooths inside and reuses the pass's norms:
  same operand as smoothing then computing the bound from scratch."""
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.kernels import k_smoothing, splash
  banner("fixed-m operand from the smoothing pass")
  q = seeded((1, 3, 400, 128), 193)
  k = seeded((1, 3, 400, 128), 194) + 1.0
  ks, kn = k_smoothing.smooth_keys(k, norms=True)
  a = splash._fixed_m_operand(q, ks, None, kn)
  b = splash._fixed_m_operand(q, ks, None)
  torch.cuda.synchronize()
  assert torch.equal(a, b)


@pytest.mark.parametrize("shape,hkv,kv_len,d", [
    ((2, 6, 700), 3, None, 128),      # GQA, (B, Hq, Sq)
    ((1, 4, 333), 4, 900, 128),       # Skv 1000 with kv_len
    ((1, 2, 500), 1, 1500, 64),
])
def test_fixed_m_prepare_matches_separate_passes(ksm, shape, hkv, kv_len, d):
  """dt_fixed_m_prepare's operand and smoothed keys equal those of the
  separate passes (smooth_keys, dt_max_row_norm and the torch operand
  arithmetic), bit for bit, with and without smoothing."""
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  b, hq, sq = shape
  skv = 1000 if kv_len is None else kv_len + 100
  banner(f"fixed_m_prepare {shape} hkv={hkv} skv={skv} kv_len={kv_len} d={d}")
  q = seeded((b, sq, hq, d), 195).transpose(1, 2)   # strided (B,S,H,D) view
  k = seeded((b, hkv, skv, d), 196) + 1.0
  ks, mk = fmb.fixed_m_prepare(q, k, kv_len=kv_len, smooth=True)
  ks2, kn = ksm.smooth_keys(k, kv_len, norms=True)
  qn = fmb.fixed_m_query_norms(q)
  want = fmb.fixed_m_operands_from_norms(
      qn, kn.repeat_interleave(hq // hkv), gate=fmb.FIXED_M_SAFE_BOUND)
  k_same, mk0 = fmb.fixed_m_prepare(q, k, smooth=False)
  want0 = fmb.fixed_m_operands_from_norms(
      qn, fmb.max_row_norm_per_head(k).repeat_interleave(hq // hkv),
      gate=fmb.FIXED_M_SAFE_BOUND)
  torch.cuda.synchronize()
  assert torch.equal(ks, ks2)
  assert torch.equal(mk, want), (mk, want)
  assert k_same is k
  assert torch.equal(mk0, want0), (mk0, want0)
  # the bound is a real bound: no scaled logit exceeds it
  c = np.log2(np.e) / np.sqrt(d)
  logits = np.einsum("bhid,bhjd->bhij", c * to64(q),
                     np.repeat(to64(ks), hq // hkv, axis=1))
  assert (np.abs(logits).max(axis=(0, 2, 3)) <= to64(mk[0]) + 1e-3).all()
