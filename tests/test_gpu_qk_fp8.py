"""qk_fp8 path on the GPU (kernels/splash.py:420-424): the saturating E4M3
cast (dt_quantize_e4m3, kernels/fp8_cast.py:28-39) bit-exact against the
oracle, and attention with E4M3 q/k in the QK product against the float64
softmax of the same E4M3-rounded operands.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A
from oracle import fp8 as P8

pytestmark = pytest.mark.gpu

LN2 = float(np.log(2.0))


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _codes(t):
  return t.view(torch.uint8).cpu().numpy()


def test_quantize_bit_exact(dta):
  from diffusers_tpu_amd.kernels.fp8_cast import quantize_saturating
  banner("quantize_saturating specials + random")
  special = torch.tensor([0.0, -0.0, 1.0, 448.0, 449.0, 464.0, 1e30, -1e30,
                          2.0**-9, 2.0**-10, 3 * 2.0**-10, 1.0625, 1.1875,
                          -2.0, 240.0, 2.0**-6, 7 * 2.0**-9, 1e-30],
                         dtype=torch.float32)
  x = seeded((2, 3, 333, 128), 100) * 30
  x.view(-1)[:special.numel()] = special.to(x.dtype)
  got = _codes(quantize_saturating(x))
  want = P8.quantize_e4m3(to64(x))
  np.testing.assert_array_equal(got, want.reshape(got.shape))


def test_quantize_strided_and_factor(dta):
  from diffusers_tpu_amd.kernels.fp8_cast import quantize_saturating
  banner("quantize_saturating strided view + factor")
  base = seeded((1, 200, 4, 64), 101) * 5
  x = base.transpose(1, 2)                 # (B, H, S, D) view of BSHD storage
  got = quantize_saturating(x, factor=0.75)
  assert got.is_contiguous() and got.shape == x.shape
  scaled = (x.float() * 0.75).to(torch.bfloat16)
  np.testing.assert_array_equal(_codes(got),
                                P8.quantize_e4m3(to64(scaled)))


def _q8k8(q, k, scale=None):
  """The operands the E4M3 QK product sees, in log2 units: q scaled by
  scale*log2(e) and rounded to bf16, then both cast to E4M3."""
  c = (1.0 / np.sqrt(q.shape[-1]) if scale is None else scale) * np.log2(np.e)
  qs = (q.float() * c).to(torch.bfloat16)
  return P8.e4m3_round(to64(qs)), P8.e4m3_round(to64(k))


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, Sq, Skv, kv_len)
    (1, 2, 2, 128, 128, None),
    (2, 3, 3, 257, 300, 211),
    (1, 4, 2, 130, 190, None),
    (1, 2, 2, 64, 4096, 4033),
    (1, 1, 1, 1, 1, None),
])
def test_attention_qk_fp8_matches_oracle(dta, case):
  b, hq, hkv, sq, skv, kv_len = case
  banner(f"attention qk_fp8 {case}")
  q = seeded((b, hq, sq, 128), 110)
  k = seeded((b, hkv, skv, 128), 111)
  v = seeded((b, hkv, skv, 128), 112)
  got = dta.attention(q, k, v, scale=None, block_q=512, block_kv=512,
                      block_kv_compute=512, qk_fp8=True, kv_len=kv_len)
  torch.cuda.synchronize()
  q8, k8 = _q8k8(q, k)
  # logits q8.k8 are already in log2 units: exp2(x) = exp(ln2 * x)
  want = A.attention_f64(q8, k8, to64(v), scale=LN2, kv_len=kv_len)
  assert_attn_close(to64(got), want, f"qk_fp8 {case}")


def test_residual_qk_fp8_and_fixed_m(dta):
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  banner("residual qk_fp8, with and without fixed-m")
  q = seeded((1, 3, 150, 128), 113)
  k = seeded((1, 3, 333, 128), 114)
  k = (k.float() - k.float().mean(dim=2, keepdim=True)).to(k.dtype)
  v = seeded((1, 3, 333, 128), 115)
  q8, k8 = _q8k8(q, k)
  wo, wm, wl = A.residual_f64(q8, k8, to64(v), scale=LN2)
  mk = fmb.fixed_m_operands_from_norms(fmb.fixed_m_query_norms(q),
                                       fmb.max_row_norm_per_head(k))
  for kw in ({}, {"use_fixed_m": True, "mk": mk}):
    o, m, l = dta.residual_attention(q, k, v, scale=None, block_q=1,
                                     block_kv=1, block_kv_compute=1,
                                     qk_fp8=True, **kw)
    torch.cuda.synchronize()
    assert_attn_close(to64(o) / to64(l), wo / wl, f"residual qk_fp8 {kw.keys()}")
    lse = to64(m) + np.log2(to64(l))
    np.testing.assert_allclose(lse.ravel(),
                               (np.asarray(wm) + np.log2(wl)).ravel(),
                               atol=2e-3)


def test_qk_fp8_error_vs_bf16_path(dta):
  """Informational bound: E4M3 logits stay close to the bf16 result on
  N(0,1) data (post-norm rows are O(1), kernels/splash.py:418-419)."""
  banner("qk_fp8 vs bf16 path")
  q = seeded((1, 4, 512, 128), 116)
  k = seeded((1, 4, 1024, 128), 117)
  v = seeded((1, 4, 1024, 128), 118)
  a = dta.attention(q, k, v, scale=None, block_q=1, block_kv=1,
                    block_kv_compute=1, qk_fp8=True)
  b = dta.attention(q, k, v, scale=None, block_q=1, block_kv=1,
                    block_kv_compute=1)
  torch.cuda.synchronize()
  err = np.abs(to64(a) - to64(b))
  assert err.mean() < 1e-2 and err.max() < 0.1
