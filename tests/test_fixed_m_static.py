"""Calibrated fixed-m operands (kernels/fixed_m_bound.py:296-408, host
logic, CPU) and the sampled max-logit measurement
(kernels/fixed_m_bound.py:169-286, GPU, against a brute-force oracle)."""
import math

import numpy as np
import pytest
import torch

from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
from oracle import fixed_m as FM
from oracle import fp8 as P8


def test_static_operands_known_answers():
  gate = fmb.FIXED_M_RING_SAFE_BOUND          # 106.5
  mk = fmb.static_fixed_m_operands([2.0, 10.0, 20.0], [3.0, 10.0, 11.0],
                                   margin_log2=1.0)
  # bounds 6, 100, 220: ceil + 1 = 7, 101, 221 against 106.5
  np.testing.assert_array_equal(mk, [[106, 106, 106], [1, 1, 0]])
  assert mk.dtype == np.float32
  # the margin decides eligibility only: 100 + 7 > 106.5
  mk = fmb.static_fixed_m_operands([10.0], [10.0], margin_log2=7.0)
  np.testing.assert_array_equal(mk, [[106], [0]])
  # E4M3 inflation (1 + 2^-4)^2: 100 -> 112.89 -> ineligible
  mk = fmb.static_fixed_m_operands([10.0], [10.0], margin_log2=0.0,
                                   qk_fp8=True)
  assert mk[1, 0] == 0 and math.isclose((1 + 2 ** -4) ** 2, 1.12890625)
  # a measured max logit tightens (min with the Cauchy-Schwarz product) ...
  mk = fmb.static_fixed_m_operands([2.0, 10.0, 20.0], [3.0, 10.0, 11.0],
                                   margin_log2=1.0,
                                   max_logit=[1.0, 50.0, 105.0])
  np.testing.assert_array_equal(mk[1], [1, 1, 1])
  # ... but never widens past it
  mk = fmb.static_fixed_m_operands([20.0], [11.0], margin_log2=0.0,
                                   max_logit=[500.0])
  assert mk[1, 0] == 0
  # the flat gate
  mk = fmb.static_fixed_m_operands([10.0], [20.0], margin_log2=0.0,
                                   gate=fmb.FIXED_M_SAFE_BOUND)
  np.testing.assert_array_equal(mk, [[213], [1]])
  # torch inputs work as well
  mk = fmb.static_fixed_m_operands(torch.tensor([2.0]), torch.tensor([3.0]),
                                   margin_log2=0.0)
  np.testing.assert_array_equal(mk, [[106], [1]])


@pytest.mark.parametrize("kwargs,exc", [
    (dict(qn_max=[1.0, 2.0], mk_h=[1.0]), ValueError),
    (dict(qn_max=[[1.0]], mk_h=[[1.0]]), ValueError),
    (dict(qn_max=[1.0], mk_h=[1.0], margin_log2=-1.0), ValueError),
    (dict(qn_max=[1.0], mk_h=[1.0], max_logit=[-1.0]), ValueError),
    (dict(qn_max=[1.0], mk_h=[1.0], max_logit=[float("nan")]), ValueError),
    (dict(qn_max=[1.0], mk_h=[1.0], max_logit=[1.0, 2.0]), ValueError),
])
def test_static_operands_errors(kwargs, exc):
  kwargs.setdefault("margin_log2", 0.0)
  with pytest.raises(exc):
    fmb.static_fixed_m_operands(**kwargs)


def test_bruteforce_oracle_pins_itself():
  """The brute-force oracle on a case with a known answer: colinear q and k
  give |q.k| = |q||k|, the Cauchy-Schwarz bound."""
  q = np.zeros((1, 1, 3, 8))
  k = np.zeros((1, 1, 2, 8))
  q[0, 0, 1, :2] = [3.0, 4.0]          # |q| = 5
  k[0, 0, 1, :2] = [-6.0, -8.0]        # |k| = 10, anti-parallel
  got = FM.max_abs_logit_bruteforce(q, k, 1.0)
  assert got[0] == 50.0
  # stride 2 skips row 1
  assert FM.max_abs_logit_bruteforce(q, k, 1.0, stride=2)[0] == 0.0


@pytest.mark.gpu
@pytest.mark.parametrize("hkv,num,fp8", [(2, 7, False), (1, 0, False),
                                         (2, 1000, True)])
def test_sampled_max_abs_logit_matches_bruteforce(hkv, num, fp8):
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from gpu_helpers import banner, seeded, to64
  banner(f"sampled_max_abs_logit hkv={hkv} num={num} fp8={fp8}")
  q = seeded((1, 2, 40, 128), 600)
  k = seeded((1, hkv, 33, 128), 601)
  got = fmb.sampled_max_abs_logit(q, k, num_samples=num, qk_fp8=fp8,
                                  rows_per_chunk=3)
  factor = 1.44269504 / math.sqrt(128)
  stride = -(-40 // (40 if num <= 0 or num >= 40 else num))
  kk = np.repeat(to64(k), 2 // hkv, axis=1)
  qq = to64(q)
  if fp8:
    # the product rounds the scaled q to bf16, then both through E4M3
    qs = FM.bf16_round(np.float32(factor) * qq.astype(np.float32))
    want = FM.max_abs_logit_bruteforce(P8.e4m3_round(qs), P8.e4m3_round(kk),
                                       1.0, stride)
  else:
    want = FM.max_abs_logit_bruteforce(qq, kk, factor, stride)
  np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-5)
  # seq_axis=1 layout gives the same
  got1 = fmb.sampled_max_abs_logit(q.transpose(1, 2), k.transpose(1, 2),
                                   seq_axis=1, num_samples=num, qk_fp8=fp8)
  np.testing.assert_allclose(got1.cpu().numpy(), got.cpu().numpy(), rtol=1e-6)
