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
