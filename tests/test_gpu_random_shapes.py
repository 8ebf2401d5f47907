"""Seeded random shapes through every attention entry point, against the
float64 oracle: dense (bf16 and E4M3 keys), residual, block-sparse, GQA,
kv_len anywhere, strided views.  The shapes are drawn once from a fixed
seed, so a failure names a reproducible case."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A
from oracle import fp8 as P8
from oracle import sparse as SP

pytestmark = pytest.mark.gpu


def _cases(n=12, seed=2026):
  rng = np.random.default_rng(seed)
  out = []
  for i in range(n):
    hkv = int(rng.choice([1, 2, 3]))
    group = int(rng.choice([1, 2, 4]))
    sq = int(rng.integers(1, 700))
    skv = int(rng.integers(1, 1500))
    kv_len = None if rng.random() < 0.4 else int(rng.integers(1, skv + 1))
    b = int(rng.choice([1, 2]))
    out.append((i, b, hkv * group, hkv, sq, skv, kv_len))
  return out


CASES = _cases()


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


@pytest.mark.parametrize("case", CASES, ids=[f"case{c[0]}" for c in CASES])
def test_random_shape(dta, case):
  i, b, hq, hkv, sq, skv, kv_len = case
  banner(f"random {case}")
  q = seeded((b, hq, sq, 128), 300 + i)
  k = seeded((b, hkv, skv, 128), 400 + i)
  v = seeded((b, hkv, skv, 128), 500 + i)
  kw = dict(scale=None, block_q=256, block_kv=256, block_kv_compute=256,
            kv_len=kv_len)
  # dense, bf16 keys
  got = dta.attention(q, k, v, **kw)
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=kv_len)
  assert_attn_close(to64(got), want, f"dense {case}")
  # strided (B,S,H,D) storage views give the same bits
  qs = q.transpose(1, 2).contiguous().transpose(1, 2)
  assert torch.equal(dta.attention(qs, k, v, **kw), got)
  # residual form
  o, m, l = dta.residual_attention(q, k, v, **kw)
  assert_attn_close(to64(o) / to64(l), want, f"residual {case}")
  # E4M3 keys
  c = np.log2(np.e) / np.sqrt(128)
  q8 = P8.e4m3_round(to64((q.float() * c).to(torch.bfloat16)))
  k8 = P8.e4m3_round(to64(k))
  got8 = dta.attention(q, k, v, qk_fp8=True, **kw)
  want8 = A.attention_f64(q8, k8, to64(v), scale=np.log(2.0), kv_len=kv_len)
  assert_attn_close(to64(got8), want8, f"qk_fp8 {case}")
  # block-sparse: a random table in 256 x 256 blocks that keeps block 0
  from diffusers_tpu_amd.kernels import sparse_splash
  rng = np.random.default_rng(i)
  nq, nk = -(-sq // 256), -(-skv // 256)
  table = [sorted({0} | set(rng.choice(nk, size=rng.integers(1, nk + 1),
                                       replace=False).tolist()))
           for _ in range(nq)]
  gots = sparse_splash.attention(q, k, v, kv_table=table, **kw)
  mask = SP.block_mask(sq, skv, 256, 256, table)
  if kv_len is not None:
    mask[:, kv_len:] = False
  wants = SP.attention_masked_f64(to64(q), to64(k), to64(v), mask)
  assert_attn_close(to64(gots), wants, f"sparse {case}")


def _large_cases(n=6, seed=2027):
  """Key lengths past the packed-V threshold, few query blocks (so the
  grid's last round splits), GQA, kv_len anywhere."""
  rng = np.random.default_rng(seed)
  out = []
  for i in range(n):
    hkv = int(rng.choice([1, 2]))
    group = int(rng.choice([1, 2]))
    sq = int(rng.integers(1, 3000))
    skv = int(rng.integers(33000, 60000))
    kv_len = None if rng.random() < 0.4 else int(rng.integers(32768, skv + 1))
    out.append((i, 1, hkv * group, hkv, sq, skv, kv_len))
  return out


LARGE = _large_cases()


@pytest.mark.parametrize("case", LARGE, ids=[f"large{c[0]}" for c in LARGE])
def test_random_large_shape(dta, case):
  """Dense, residual and E4M3-key attention at lengths that take packed V
  and the tail split, on sampled query rows (first, middle, last) against
  the float64 oracle."""
  i, b, hq, hkv, sq, skv, kv_len = case
  banner(f"random large {case}")
  q = seeded((b, hq, sq, 128), 600 + i)
  k = seeded((b, hkv, skv, 128), 700 + i)
  v = seeded((b, hkv, skv, 128), 800 + i)
  kw = dict(scale=None, block_q=256, block_kv=256, block_kv_compute=256,
            kv_len=kv_len)
  rows = np.unique(np.r_[0:min(sq, 8), sq // 2, max(sq - 8, 0):sq])
  got = dta.attention(q, k, v, **kw)
  o, m, l = dta.residual_attention(q, k, v, **kw)
  got8 = dta.attention(q, k, v, qk_fp8=True, **kw)
  torch.cuda.synchronize()
  want = A.attention_rows_f64(to64(q), to64(k), to64(v), rows, kv_len=kv_len)
  assert_attn_close(to64(got)[:, :, rows], want, f"dense {case}")
  assert_attn_close((to64(o) / to64(l))[:, :, rows], want, f"residual {case}")
  c = np.log2(np.e) / np.sqrt(128)
  q8 = P8.e4m3_round(to64((q[:, :, rows].float() * c).to(torch.bfloat16)))
  k8 = P8.e4m3_round(to64(k))
  want8 = A.attention_f64(q8, k8, to64(v), scale=np.log(2.0), kv_len=kv_len)
  assert_attn_close(to64(got8)[:, :, rows], want8, f"qk_fp8 {case}")


def _dim_cases(n=10, seed=2028):
  """Head dims 8..128 (multiples of 8: the D = 64 kernel, the D = 128
  kernel and zero-padded dims of both), fp32 / fp16 / bf16 inputs, fixed-m
  on and off."""
  rng = np.random.default_rng(seed)
  out = []
  for i in range(n):
    d = int(rng.integers(1, 17)) * 8
    hkv = int(rng.choice([1, 2]))
    group = int(rng.choice([1, 3]))
    sq = int(rng.integers(1, 600))
    skv = int(rng.integers(1, 1200))
    kv_len = None if rng.random() < 0.5 else int(rng.integers(1, skv + 1))
    dtype = str(rng.choice(["bfloat16", "float16", "float32"]))
    fixed = bool(rng.random() < 0.5)
    out.append((i, d, hkv * group, hkv, sq, skv, kv_len, dtype, fixed))
  return out


DIMS = _dim_cases()


@pytest.mark.parametrize("case", DIMS, ids=[f"dim{c[0]}" for c in DIMS])
def test_random_head_dim(dta, case):
  """Normalized and residual attention at random head dims and input
  dtypes against the float64 oracle of the bf16-rounded inputs; the output
  comes back in the input dtype."""
  i, d, hq, hkv, sq, skv, kv_len, dtype, fixed = case
  banner(f"random dim {case}")
  dt = getattr(torch, dtype)
  q = seeded((1, hq, sq, d), 900 + i, dtype=dt)
  k = seeded((1, hkv, skv, d), 1000 + i, dtype=dt)
  v = seeded((1, hkv, skv, d), 1100 + i, dtype=dt)
  kw = dict(scale=None, block_q=256, block_kv=256, block_kv_compute=256,
            kv_len=kv_len)
  got = dta.attention(q, k, v, use_fixed_m=fixed, **kw)
  assert got.dtype == dt and got.shape == q.shape
  # the kernels read bf16: the oracle sees the same rounded inputs
  r = lambda t: to64(t.to(torch.bfloat16))
  want = A.attention_f64(r(q), r(k), r(v), kv_len=kv_len)
  assert_attn_close(to64(got), want, f"dense {case}")
  o, m, l = dta.residual_attention(q, k, v, **kw)
  assert o.shape == q.shape and m.shape == q.shape[:3] + (1,)
  assert_attn_close(to64(o) / to64(l), want, f"residual {case}")
  # E4M3 keys at this head dim (runs zero-padded to 128 channels, with the
  # scale of the real dim)
  c = np.log2(np.e) / np.sqrt(d)
  qb = q.to(torch.bfloat16)
  q8 = P8.e4m3_round(to64((qb.float() * c).to(torch.bfloat16)))
  k8 = P8.e4m3_round(r(k))
  got8 = dta.attention(q, k, v, qk_fp8=True, **kw)
  want8 = A.attention_f64(q8, k8, r(v), scale=np.log(2.0), kv_len=kv_len)
  assert_attn_close(to64(got8), want8, f"qk_fp8 {case}")
