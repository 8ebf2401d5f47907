"""Parity of the gfx950 flash-attention kernel (dt_flash_fwd via the C ABI)
against the float64 oracle (oracle/attention.py), on seeded inputs.

Edge cases follow what the reference's kernel handles: ragged key lengths
that are not a tile multiple (kernels/splash.py:281-306), runtime kv_len
masking (:216-218, :277-331), Sq != Skv, GQA (:438-444), strided inputs,
and the residual (o, m, l) form (:665-742).
"""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _run(dta, q, k, v, **kw):
  out = dta.attention(q, k, v, scale=kw.pop("scale", None), block_q=512,
                      block_kv=512, block_kv_compute=512, **kw)
  torch.cuda.synchronize()
  return out


CASES = [
    # (B, Hq, Hkv, Sq, Skv, D, kv_len)
    (1, 8, 8, 1024, 1024, 64, None),     # plumbing shape
    (1, 2, 2, 128, 128, 128, None),      # one tile pair
    (1, 2, 2, 100, 77, 128, None),       # ragged Sq and Skv
    (2, 3, 3, 257, 300, 128, 211),       # batch, kv_len inside a tile
    (1, 2, 2, 64, 4096, 128, 4033),      # long keys, kv_len mid-tile
    (1, 4, 2, 130, 190, 128, None),      # GQA 2:1
    (1, 1, 1, 1, 1, 128, None),          # single query, single key
    (1, 2, 2, 33, 65, 64, 64),           # kv_len at a tile boundary
]


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_attention_matches_oracle(dta, case):
  b, hq, hkv, sq, skv, d, kv_len = case
  banner(f"attention {case}")
  q = seeded((b, hq, sq, d), 10)
  k = seeded((b, hkv, skv, d), 11)
  v = seeded((b, hkv, skv, d), 12)
  out = _run(dta, q, k, v, kv_len=kv_len)
  assert out.shape == q.shape and out.dtype == torch.bfloat16
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=kv_len)
  assert_attn_close(to64(out), want, str(case))


def test_attention_fp32_inputs_and_scale(dta):
  banner("attention fp32 in/out, explicit scale")
  q = seeded((1, 2, 200, 64), 20, dtype=torch.float32)
  k = seeded((1, 2, 150, 64), 21, dtype=torch.float32)
  v = seeded((1, 2, 150, 64), 22, dtype=torch.float32)
  out = _run(dta, q, k, v, scale=0.2)
  assert out.dtype == torch.float32
  # the kernel computes on bf16 operands (as the reference casts q and
  # feeds bf16 k/v, kernels/splash.py:633); compare with fp32 oracle inputs
  want = A.attention_f64(to64(q), to64(k), to64(v), scale=0.2)
  assert_attn_close(to64(out), want, "fp32")


def test_attention_strided_views(dta):
  """q/k/v as (B,S,H,D) storage viewed as (B,H,S,D)."""
  banner("attention strided views")
  qs = seeded((2, 300, 4, 128), 30)
  ks = seeded((2, 280, 4, 128), 31)
  vs = seeded((2, 280, 4, 128), 32)
  q, k, v = (t.transpose(1, 2) for t in (qs, ks, vs))
  out = _run(dta, q, k, v, kv_len=250)
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=250)
  assert_attn_close(to64(out), want, "strided")


def test_kv_len_tensor_and_padding_independence(dta):
  banner("attention kv_len tensor / pad content")
  q = seeded((1, 2, 96, 128), 40)
  k = seeded((1, 2, 512, 128), 41)
  v = seeded((1, 2, 512, 128), 42)
  a = _run(dta, q, k, v, kv_len=torch.tensor(300))
  k2, v2 = k.clone(), v.clone()
  k2[:, :, 300:] = 1e4   # garbage past kv_len must not matter
  v2[:, :, 300:] = -7.0
  b = _run(dta, q, k2, v2, kv_len=300)
  assert torch.equal(a, b)
  c = _run(dta, q, k[:, :, :300].contiguous(), v[:, :, :300].contiguous())
  assert torch.equal(a, c)


def test_residual_outputs(dta):
  banner("residual attention")
  q = seeded((1, 3, 150, 128), 50)
  k = seeded((1, 3, 333, 128), 51)
  v = seeded((1, 3, 333, 128), 52)
  o, m, l = dta.residual_attention(q, k, v, scale=None, block_q=1,
                                   block_kv=1, block_kv_compute=1)
  torch.cuda.synchronize()
  wo, wm, wl = A.residual_f64(to64(q), to64(k), to64(v))
  # m is the scale reference of o and l (kernels/splash.py:665-742 allows a
  # bound instead of the row max; merges are LSE-space): the m-invariant
  # lse = m + log2(l) must match, and m must sit within 2^13 of the max.
  # The kernel folds scale*log2(e) into q and rounds that to bf16 (as
  # kernels/splash.py:607-609 does), which moves each log2-domain logit by at
  # most 2^-9 * sum_d |c q_d k_d|: the bound `shift` below, per row.
  c = np.log2(np.e) / np.sqrt(128.0)
  shift = 2.0**-9 * np.einsum("bhid,bhjd->bhij", np.abs(c * to64(q)),
                              np.abs(to64(k))).max(-1)
  shift = shift.ravel()
  gm, gl, wm1, wl1 = (np.ravel(to64(t) if torch.is_tensor(t) else t)
                      for t in (m, l, wm, wl))
  err = np.abs(gm + np.log2(gl) - (wm1 + np.log2(wl1)))
  assert (err <= shift + 1e-3).all(), float((err - shift).max())
  assert (gm <= wm1 + shift + 1e-4).all() and (gm >= wm1 - 13).all()
  assert_attn_close(to64(o) / to64(l), wo / wl, "residual o/l")
  # shards merged in LSE space reproduce the one-pass result
  parts = [dta.residual_attention(q, k[:, :, a:b_].contiguous(),
                                  v[:, :, a:b_].contiguous(), scale=None,
                                  block_q=1, block_kv=1, block_kv_compute=1)
           for a, b_ in ((0, 100), (100, 333))]
  from diffusers_tpu_amd.kernels.splash import merge_residuals
  merged = merge_residuals(parts)
  assert_attn_close(to64(merged), wo / wl, "merged")


def test_errors_raise(dta):
  q = seeded((1, 2, 8, 128), 1)
  with pytest.raises(ValueError):
    _run(dta, q, q, q, kv_len=9)
  x = seeded((1, 2, 8, 100), 1)              # not a multiple of 8
  with pytest.raises(NotImplementedError):
    _run(dta, x, x, x)
  x = seeded((1, 2, 8, 264), 1)              # above the kernels' 256
  with pytest.raises(NotImplementedError):
    _run(dta, x, x, x)


@pytest.mark.parametrize("d", [32, 72, 96, 120])
def test_other_head_dims_by_zero_padding(dta, d):
  """Head dims below 128 run on the 64/128 kernels with zero-padded
  channels; the softmax scale stays 1/sqrt(d)."""
  banner(f"attention head_dim {d}")
  q = seeded((1, 3, 150, d), 160)
  k = seeded((1, 3, 210, d), 161)
  v = seeded((1, 3, 210, d), 162)
  out = _run(dta, q, k, v, kv_len=199)
  assert out.shape == q.shape
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=199)
  assert_attn_close(to64(out), want, f"d={d}")
  o, m, l = dta.residual_attention(q, k, v, scale=None, block_q=1,
                                   block_kv=1, block_kv_compute=1, kv_len=199)
  assert o.shape == q.shape
  assert_attn_close(to64(o) / to64(l), want, f"residual d={d}")
  from oracle import fp8 as P8
  c = np.log2(np.e) / np.sqrt(d)
  q8 = P8.e4m3_round(to64((q.float() * c).to(torch.bfloat16)))
  got8 = _run(dta, q, k, v, kv_len=199, qk_fp8=True)
  want8 = A.attention_f64(q8, P8.e4m3_round(to64(k)), to64(v),
                          scale=np.log(2.0), kv_len=199)
  assert_attn_close(to64(got8), want8, f"qk_fp8 d={d}")


def test_softmax_extremes(dta):
  """Large logits (|s| ~ 1e3) stay finite and exact-ish: online max."""
  banner("attention extreme logits")
  q = seeded((1, 1, 64, 128), 60) * 30
  k = seeded((1, 1, 200, 128), 61) * 3
  v = seeded((1, 1, 200, 128), 62)
  out = _run(dta, q, k, v)
  want = A.attention_f64(to64(q), to64(k), to64(v))
  # near one-hot rows: error dominated by bf16 logit rounding of huge values
  got = to64(out)
  assert np.isfinite(got).all()
  assert np.abs(got - want).mean() < 5e-2


def test_sdpa_adapter(dta):
  """kernels/mesh_attention.py::configure's SDPA-shaped callable."""
  banner("sdpa adapter")
  from diffusers_tpu_amd.kernels import mesh_attention
  sdpa = mesh_attention.configure()
  q = seeded((1, 4, 100, 128), 70)
  k = seeded((1, 4, 120, 128), 71)
  v = seeded((1, 4, 120, 128), 72)
  a = sdpa(q, k, v)
  b = _run(dta, q, k, v)
  assert torch.equal(a, b)
  # k-smoothing (softmax-invariant) stays within tolerance of the oracle
  smooth = mesh_attention.configure(k_smoothing=True)
  c = smooth(q, k, v, kv_len=111)
  torch.cuda.synchronize()
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=111)
  assert_attn_close(to64(c), want, "k-smoothed")
  with pytest.raises(NotImplementedError):
    sdpa(q, k, v, is_causal=True)
  with pytest.raises(ValueError):
    sdpa(q, k[:, :2], v[:, :2])


@pytest.mark.parametrize("d", [64, 128])
def test_out_with_8_byte_aligned_rows(dta, d):
  """``out=`` views the ABI accepts (8-byte aligned rows: a pointer 8 bytes
  past 16-byte alignment, or a row stride of d + 4 elements) get the same
  bits as a fresh output."""
  banner(f"out= alignment d={d}")
  q = seeded((1, 3, 300, d), 90)
  k = seeded((1, 3, 333, d), 91)
  v = seeded((1, 3, 333, d), 92)
  want = _run(dta, q, k, v)
  flat = torch.zeros(q.numel() + 4, device="cuda", dtype=torch.bfloat16)
  shifted = flat[4:].view(q.shape)
  assert shifted.data_ptr() % 16 == 8
  wide = torch.zeros((1, 3, 300, d + 4), device="cuda",
                     dtype=torch.bfloat16)[..., :d]
  for out in (shifted, wide):
    got = dta.attention(q, k, v, scale=None, block_q=512, block_kv=512,
                        block_kv_compute=512, out=out)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    assert torch.equal(got, want)
