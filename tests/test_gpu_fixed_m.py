"""Fixed-m softmax path on the GPU: the per-head row-norm reduction
(dt_max_row_norm, kernels/fixed_m_bound.py:57-118) against the oracle, and
attention with the fixed-m operand (kernels/splash.py:170-248) against the
float64 dense softmax.

That the kernel really ran fixed-m is visible in the residual form: a fixed
head's m stays at mk[0, h] - 88 (no re-base fires for a bound-respecting
head), where the online path would report m near the row max.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A
from oracle import fixed_m as F

pytestmark = pytest.mark.gpu

C = float(np.log2(np.e))


@pytest.fixture(scope="module")
def fmb():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.kernels import fixed_m_bound
  return fixed_m_bound


@pytest.mark.parametrize("shape,seq_axis,d", [
    ((2, 3, 1000, 128), 2, 128),   # (B, H, S, D), ragged S
    ((1, 777, 4, 64), 1, 64),      # (B, S, H, D) storage
    ((1, 5, 70, 128), 2, 128),     # fewer rows than one load step
])
def test_max_row_norm_matches_oracle(fmb, shape, seq_axis, d):
  banner(f"max_row_norm {shape} seq_axis={seq_axis}")
  x = seeded(shape, 80) * 3
  got = fmb.max_row_norm_per_head(x, seq_axis=seq_axis)
  xb = to64(x) if seq_axis == 2 else to64(x).transpose(0, 2, 1, 3)
  want = F.max_row_norm_per_head(xb)
  np.testing.assert_allclose(to64(got), want, rtol=2e-6)


def test_max_row_norm_strided_factor_and_accumulate(fmb):
  banner("max_row_norm strided view, factor, accumulate")
  base = seeded((2, 300, 6, 128), 81)
  x = base[:, :, 1:5].transpose(1, 2)         # (B, 4, S, D) view, strided
  want = F.max_row_norm_per_head(to64(x))
  got = fmb.max_row_norm_per_head(x, factor=0.25)
  np.testing.assert_allclose(to64(got), 0.25 * want, rtol=2e-6)
  # folding a second shard into the same output keeps the larger maximum
  y = seeded((2, 4, 50, 128), 82) * 10
  fmb.max_row_norm_per_head(y, out=got, factor=0.25)
  both = np.maximum(want, F.max_row_norm_per_head(to64(y)))
  np.testing.assert_allclose(to64(got), 0.25 * both, rtol=2e-6)


def test_fixed_m_operands_match_oracle(fmb):
  banner("fixed_m_operands")
  q = seeded((1, 4, 500, 128), 83)
  k = seeded((1, 4, 500, 128), 84)
  q[:, 3] *= 12                                # head 3 over the gate
  qs = q.float() * (C / np.sqrt(128))
  got = to64(fmb.fixed_m_operands(qs, k, gate=fmb.FIXED_M_SAFE_BOUND))
  want = F.fixed_m_operands(to64(qs.to(torch.bfloat16)), to64(k))
  np.testing.assert_array_equal(got[1], want[1])
  assert (np.abs(got[0] - want[0]) <= 1).all()
  assert got[1].tolist() == [1, 1, 1, 0]


def _smoothed(k):
  """k-smoothing (softmax-invariant), as callers of fixed-m do
  (kernels/mesh_attention.py:234-236)."""
  return (k.float() - k.float().mean(dim=2, keepdim=True)).to(k.dtype)


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, Sq, Skv, kv_len, q_gain, D)
    (1, 4, 4, 300, 700, None, 1.0, 128),
    (2, 4, 2, 130, 333, 301, 1.0, 128),     # GQA, kv_len mid-tile
    (1, 2, 2, 64, 2048, None, 3.0, 128),    # larger logits, still eligible
    (2, 4, 2, 300, 1000, 901, 1.0, 64),     # head dim 64
])
def test_attention_fixed_m_matches_oracle(case):
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd as dta
  b, hq, hkv, sq, skv, kv_len, gain, d = case
  banner(f"attention use_fixed_m {case}")
  q = seeded((b, hq, sq, d), 90) * gain
  k = _smoothed(seeded((b, hkv, skv, d), 91))
  v = seeded((b, hkv, skv, d), 92)
  got = dta.attention(q, k, v, scale=None, block_q=512, block_kv=512,
                      block_kv_compute=512, use_fixed_m=True, kv_len=kv_len)
  torch.cuda.synchronize()
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=kv_len)
  assert_attn_close(to64(got), want, f"fixed-m {case}")
  online = dta.attention(q, k, v, scale=None, block_q=512, block_kv=512,
                         block_kv_compute=512, kv_len=kv_len)
  assert_attn_close(to64(got), to64(online), "fixed vs online")


@pytest.mark.parametrize("d", [128, 64])
def test_residual_fixed_m_uses_the_bound(fmb, d):
  import diffusers_tpu_amd as dta
  from diffusers_tpu_amd.kernels.splash import merge_residuals
  banner(f"residual attention with fixed-m operand, head dim {d}")
  q = seeded((1, 3, 150, d), 93)
  k = _smoothed(seeded((1, 3, 333, d), 94))
  v = seeded((1, 3, 333, d), 95)
  q[:, 2] *= 40                                # head 2 falls back online
  qn = fmb.fixed_m_query_norms(q)
  kn = fmb.max_row_norm_per_head(k)
  mk = fmb.fixed_m_operands_from_norms(qn, kn)
  assert to64(mk[1]).tolist() == [1, 1, 0]
  o, m, l = dta.residual_attention(q, k, v, scale=None, block_q=1,
                                   block_kv=1, block_kv_compute=1,
                                   use_fixed_m=True, mk=mk)
  torch.cuda.synchronize()
  gm = to64(m)[0, :, :, 0]
  fixed_m = to64(mk[0])[:2] - 88.0
  assert (gm[:2] == fixed_m[:, None]).all(), "fixed heads re-based"
  wo, wm, wl = A.residual_f64(to64(q), to64(k), to64(v))
  assert_attn_close((to64(o) / to64(l))[:, :2], (wo / wl)[:, :2],
                    "fixed residual o/l")
  # head 2 (flag 0) runs the online path: bit-identical to a call without mk
  o2, m2, l2 = dta.residual_attention(q, k, v, scale=None, block_q=1,
                                      block_kv=1, block_kv_compute=1)
  for a, b_ in ((o, o2), (m, m2), (l, l2)):
    assert torch.equal(a[:, 2], b_[:, 2])
  assert not torch.equal(m[:, :2], m2[:, :2])
  # ring operand (one constant m for every head) over two K shards
  parts = []
  for a, b_ in ((0, 100), (100, 333)):
    ks, vs = k[:, :, a:b_].contiguous(), v[:, :, a:b_].contiguous()
    rk = fmb.ring_fixed_m_operands(qn, fmb.max_row_norm_per_head(ks))
    parts.append(dta.residual_attention(q, ks, vs, scale=None, block_q=1,
                                        block_kv=1, block_kv_compute=1,
                                        use_fixed_m=True, mk=rk))
  assert_attn_close(to64(merge_residuals(parts))[:, :2], (wo / wl)[:, :2],
                    "ring fixed-m merge")


@pytest.mark.parametrize("d", [96, 32])
def test_fixed_m_other_head_dims(d):
  """use_fixed_m with a head dim the kernels take zero-padded: the bound is
  computed on the padded tensors (zero channels change no norm)."""
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd as dta
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  banner(f"fixed-m head dim {d}")
  q = seeded((1, 2, 200, d), 97)
  k = _smoothed(seeded((1, 2, 300, d), 98))
  v = seeded((1, 2, 300, d), 99)
  got = dta.attention(q, k, v, scale=None, block_q=0, block_kv=0,
                      block_kv_compute=0, use_fixed_m=True, kv_len=280)
  torch.cuda.synchronize()
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=280)
  assert_attn_close(to64(got), want, f"fixed-m d={d}")
  qs = q.float() * (C / np.sqrt(d))
  mk = fmb.fixed_m_prepare(q, k, smooth=False)[1]
  want_mk = F.fixed_m_operands(to64(qs.to(torch.bfloat16)), to64(k))
  np.testing.assert_array_equal(to64(mk[1]), want_mk[1])
  assert (np.abs(to64(mk[0]) - want_mk[0]) <= 1).all()
  ks, _ = fmb.fixed_m_prepare(q, k, kv_len=280, smooth=True)
  assert ks.shape == k.shape
