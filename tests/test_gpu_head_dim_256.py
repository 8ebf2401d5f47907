"""Head dims above 128 (flash_wide_kernel, head dim 256; 136..248 run
zero-padded to it).  The reference's kernel takes any head dim that is a
multiple of 8 (kernels/splash.py:156-160); every case here is checked
against the float64 oracle at the north-star tolerance."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A
from oracle import fixed_m as FM

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sp():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.kernels import splash
  return splash


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, Sq, Skv, D, kv_len)
    (1, 2, 2, 128, 128, 256, None),
    (2, 4, 2, 300, 1000, 256, 777),
    (1, 3, 1, 129, 33, 256, 31),
    (1, 2, 2, 257, 700, 192, None),
    (2, 1, 1, 64, 900, 136, 450),
    (1, 1, 1, 1, 1, 256, None),
])
def test_attention_wide_head_dims(sp, case):
  b, hq, hkv, sq, skv, d, n = case
  banner(f"head dim {d}: {case}")
  q = seeded((b, hq, sq, d), 501)
  k = seeded((b, hkv, skv, d), 502)
  v = seeded((b, hkv, skv, d), 503)
  got = sp.attention(q, k, v, kv_len=n)
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=n)
  assert got.shape == q.shape
  assert_attn_close(to64(got), want, f"D={d} {case}")


def test_residual_wide_and_row_reference(sp):
  """Residual outputs at head dim 256: o / l against the oracle, and m the
  row reference the kernel documents (rowmax - 13 < m <= rowmax, log2
  units), so LSE merges of shards hold."""
  b, h, sq, skv, d = 1, 2, 200, 1500, 256
  banner("residual head dim 256")
  q = seeded((b, h, sq, d), 511)
  k = seeded((b, h, skv, d), 512)
  v = seeded((b, h, skv, d), 513)
  o, m, l = sp.residual_attention(q, k, v)
  wo, wm, wl = A.residual_f64(to64(q), to64(k), to64(v))
  assert_attn_close(to64(o) / to64(l), wo / wl, "residual o/l")
  # (the kernel's scores use q rounded to bf16 after scaling: they sit
  # within about 0.01 of the float64 ones)
  gm = to64(m)
  assert (gm <= wm + 2e-2).all() and (gm > wm - 13 - 2e-2).all()
  # the LSE merge of two key halves equals the whole call
  o1, m1, l1 = sp.residual_attention(q, k[:, :, :700], v[:, :, :700])
  o2, m2, l2 = sp.residual_attention(q, k[:, :, 700:], v[:, :, 700:])
  merged = sp.merge_residuals([(o1, m1, l1), (o2, m2, l2)])
  assert_attn_close(to64(merged), wo / wl, "merged halves")


def test_wide_device_lengths_and_fixed_m(sp):
  """Per-sample device lengths (one of them 0) and the fixed-m operand at
  head dim 256."""
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  b, h, s, d = 2, 2, 1200, 256
  banner("head dim 256: device lengths, fixed-m")
  q = seeded((b, h, s, d), 521)
  k = seeded((b, h, s, d), 522)
  v = seeded((b, h, s, d), 523)
  lens = torch.tensor([1100, 0], device="cuda", dtype=torch.int32)
  got = sp.attention(q, k, v, kv_len=lens)
  want = A.attention_f64(to64(q[:1]), to64(k[:1]), to64(v[:1]), kv_len=1100)
  assert_attn_close(to64(got[:1]), want, "device length 1100")
  assert not got[1].any()
  # fixed-m: the operand over smoothed keys, then attention and residual
  ks, mk = fmb.fixed_m_prepare(q, k, smooth=True)
  assert bool((mk[1] == 1).all())
  want = A.attention_f64(to64(q), to64(ks), to64(v))
  got = sp.attention(q, ks, v, use_fixed_m=True)
  assert_attn_close(to64(got), want, "fixed-m")
  o, m, l = sp.residual_attention(q, ks, v, use_fixed_m=True, mk=mk)
  assert_attn_close(to64(o) / to64(l), want, "fixed-m residual")
  fixed_m = (mk[0] - 88.0).view(1, h, 1, 1).expand_as(m)
  assert torch.equal(m, fixed_m.to(m.dtype))


def test_wide_helpers_against_the_oracle(sp):
  """Key smoothing and the row-norm reduction at head dim 256."""
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  from diffusers_tpu_amd.kernels import k_smoothing
  from diffusers_tpu_amd.kernels.block_sizes import launch_plan
  b, h, s, d, n = 1, 3, 2000, 256, 1777
  banner("head dim 256: smoothing, row norms, plan")
  k = seeded((b, h, s, d), 531)
  ks = k_smoothing.smooth_keys(k, n)
  want, mean = FM.smooth_keys(to64(k), n)
  diff = np.abs(to64(ks) - want)
  assert (diff <= 2.0 ** -8 * (np.abs(mean) + np.abs(want)) + 1e-30).all()
  norms = fmb.max_row_norm_per_head(k)
  np.testing.assert_allclose(norms.cpu().numpy(),
                             FM.max_row_norm_per_head(to64(k)), rtol=2e-6)
  plan = launch_plan(batch=2, heads=3, seq_len=1000, head_dim=256)
  assert plan.query_blocks == 2 * 3 * 8 and plan.split_parts == 1
  assert plan.key_tiles == (1000 + 31) // 32 and plan.workspace_bytes == 0
