"""Pins the CPU oracle (oracle/) against facts fixed outside its own formulas.

Each oracle function is checked against at least one of: an independent
library routine (torch SDPA, torch rms_norm, numpy complex arithmetic),
brute-force loops on tiny inputs, closed-form known answers, and invariants
that a dropped term / wrong sign / transposed operand would break.  The
reference ships no golden vectors for this path (it has no test suite), so
these are the anchors.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import fixed_m as FM
from oracle import fp8 as P8
from oracle import sparse as SP
from oracle import norm_rope as NR

RNG = np.random.default_rng(1234)


def _rand(*shape):
  return RNG.standard_normal(shape)


# ----------------------------------------------------------------- attention
def _brute_attention(q, k, v, scale, n):
  b, h, sq, d = q.shape
  out = np.zeros((b, h, sq, v.shape[-1]))
  for bi in range(b):
    for hi in range(h):
      for i in range(sq):
        logits = [sum(q[bi, hi, i, c] * k[bi, hi, j, c] for c in range(d)) * scale
                  for j in range(n)]
        mx = max(logits)
        w = [math.exp(x - mx) for x in logits]
        z = sum(w)
        for j in range(n):
          out[bi, hi, i] += w[j] / z * v[bi, hi, j]
  return out


def test_attention_matches_brute_force_tiny():
  q, k, v = _rand(1, 2, 3, 4), _rand(1, 2, 5, 4), _rand(1, 2, 5, 4)
  got = A.attention_f64(q, k, v, kv_len=4)
  want = _brute_attention(q, k, v, 1 / 2.0, 4)
  np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_attention_matches_torch_sdpa_with_mask():
  q, k, v = _rand(2, 3, 40, 16), _rand(2, 3, 50, 16), _rand(2, 3, 50, 16)
  got = A.attention_f64(q, k, v, kv_len=37, scale=0.3)
  mask = torch.arange(50) < 37
  want = torch.nn.functional.scaled_dot_product_attention(
      torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
      attn_mask=mask[None, None, None, :], scale=0.3).numpy()
  np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)


def test_attention_invariants():
  q, k, v = _rand(1, 2, 8, 16), _rand(1, 2, 12, 16), _rand(1, 2, 12, 16)
  base = A.attention_f64(q, k, v)
  # a key permutation (applied to k and v alike) changes nothing
  perm = RNG.permutation(12)
  np.testing.assert_allclose(A.attention_f64(q, k[:, :, perm], v[:, :, perm]),
                             base, atol=1e-12)
  # masking == truncation
  np.testing.assert_allclose(A.attention_f64(q, k, v, kv_len=7),
                             A.attention_f64(q, k[:, :, :7], v[:, :, :7]),
                             atol=1e-12)
  # zero query -> uniform average of the valid values
  z = A.attention_f64(np.zeros_like(q), k, v, kv_len=5)
  np.testing.assert_allclose(z, np.broadcast_to(v[:, :, :5].mean(2, keepdims=True),
                                                z.shape), atol=1e-12)
  # a single key returns its value
  one = A.attention_f64(q, k, v, kv_len=1)
  np.testing.assert_allclose(one, np.broadcast_to(v[:, :, :1], one.shape),
                             atol=1e-12)
  # adding a per-head constant vector to every key (k-smoothing in reverse)
  # is a per-row logit shift: softmax-invariant
  shift = _rand(1, 2, 1, 16)
  np.testing.assert_allclose(A.attention_f64(q, k + shift, v), base, atol=1e-10)


def test_attention_gqa_head_map():
  q, k, v = _rand(1, 4, 6, 8), _rand(1, 2, 9, 8), _rand(1, 2, 9, 8)
  got = A.attention_f64(q, k, v)
  want = A.attention_f64(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1))
  np.testing.assert_allclose(got, want, atol=1e-12)
  with pytest.raises(ValueError):
    A.attention_f64(_rand(1, 3, 2, 8), k, v)


def test_residual_form_and_lse_merge():
  q, k, v = _rand(1, 2, 10, 16), _rand(1, 2, 30, 16), _rand(1, 2, 30, 16)
  o, m, l = A.residual_f64(q, k, v)
  # LOG2_E is the reference's 9-digit constant, so exp2(s*LOG2_E) differs
  # from exp(s) at the 1e-9 level
  np.testing.assert_allclose(o / l, A.attention_f64(q, k, v), atol=1e-8)
  # m is the row max of the log2-scaled logits
  s = np.einsum("bhqd,bhkd->bhqk", q, k) / 4.0 * A.LOG2_E
  np.testing.assert_allclose(m[..., 0], s.max(-1), atol=1e-12)
  # merging two KV shards in LSE space == one pass over all keys
  o1, m1, l1 = A.residual_f64(q, k[:, :, :13], v[:, :, :13])
  o2, m2, l2 = A.residual_f64(q, k[:, :, 13:], v[:, :, 13:])
  big = np.maximum(m1, m2)
  oo = np.exp2(m1 - big) * o1 + np.exp2(m2 - big) * o2
  ll = np.exp2(m1 - big) * l1 + np.exp2(m2 - big) * l2
  np.testing.assert_allclose(oo / ll, A.attention_f64(q, k, v), atol=1e-8)


def test_attention_torch_f32_leg_agrees():
  q, k, v = (torch.randn(1, 4, 64, 32) for _ in range(3))
  got = A.attention_torch_f32(q, k, v, kv_len=50).numpy()
  want = A.attention_f64(q.numpy(), k.numpy(), v.numpy(), kv_len=50)
  np.testing.assert_allclose(got, want, atol=2e-6)


def test_attention_rows_subset():
  q, k, v = _rand(1, 2, 20, 8), _rand(1, 2, 20, 8), _rand(1, 2, 20, 8)
  rows = np.array([0, 7, 19])
  np.testing.assert_allclose(A.attention_rows_f64(q, k, v, rows),
                             A.attention_f64(q, k, v)[:, :, rows], atol=1e-12)


# ------------------------------------------------------------------- rmsnorm
def test_rms_norm_matches_torch_and_known_answer():
  x, w = _rand(3, 5, 64), 1 + 0.1 * _rand(64)
  got = NR.rms_norm_f64(x, w, 1e-6)
  want = torch.nn.functional.rms_norm(torch.from_numpy(x), (64,),
                                      torch.from_numpy(w), eps=1e-6).numpy()
  np.testing.assert_allclose(got, want, rtol=1e-12)
  # constant row c: output = w * c / sqrt(c^2 + eps)
  c = -3.0
  got = NR.rms_norm_f64(np.full((1, 8), c), np.arange(1, 9.0), 0.5)
  np.testing.assert_allclose(got[0], np.arange(1, 9.0) * c / math.sqrt(9.5))


# ---------------------------------------------------------------------- rope
def test_rope_freqs_h3_table():
  # H3 rope_angles (jax_dit.py:603-617): inv = theta^(-arange(0,32,2)/32)
  # shared by three axes -> the same 16 values three times
  f = NR.rope_freqs((32, 32, 32), 10000.0)
  one = 1.0 / 10000.0 ** (np.arange(0, 32, 2) / 32)
  np.testing.assert_allclose(f, np.tile(one, 3), rtol=1e-15)
  assert list(NR.rope_pair_axis((44, 42, 42))[[0, 21, 22, 42, 43, 63]]) == \
      [0, 0, 1, 1, 2, 2]


def test_rope_known_answer():
  # one pair, angle exactly 1 rad: (1, 0) -> (cos 1, sin 1)
  ang = NR.rope_angles_f64(np.array([[1, 0, 0]]), (2, 0, 0), 10000.0)
  assert ang[0, 0] == 1.0
  for mode in ("half", "pair"):
    out = NR.apply_rope_f64(np.array([[1.0, 0.0]]), ang, mode)
    np.testing.assert_allclose(out[0], [math.cos(1), math.sin(1)], rtol=1e-15)


def _as_complex_rotation(x, ang, mode):
  z_pairs = []
  half = ang.shape[-1]
  if mode == "half":
    z = x[..., :half] + 1j * x[..., half:2 * half]
  else:
    z = x[..., 0:2 * half:2] + 1j * x[..., 1:2 * half:2]
  z = z * np.exp(1j * ang)
  out = x.copy()
  if mode == "half":
    out[..., :half], out[..., half:2 * half] = z.real, z.imag
  else:
    out[..., 0:2 * half:2], out[..., 1:2 * half:2] = z.real, z.imag
  return out


@pytest.mark.parametrize("mode", ["half", "pair"])
@pytest.mark.parametrize("dims", [(32, 32, 32), (44, 42, 42), (0, 64, 64),
                                  (16, 56, 56)])
def test_rope_is_complex_rotation(mode, dims):
  pos = RNG.integers(-5, 90, size=(7, 3))
  x = _rand(2, 7, 128)
  ang = NR.rope_angles_f64(pos, dims, 10000.0)
  got = NR.apply_rope_f64(x, ang, mode)
  np.testing.assert_allclose(got, _as_complex_rotation(x, ang, mode),
                             atol=1e-12)
  # pass-through channels untouched, pair norms preserved, pos 0 = identity
  rot = sum(dims)
  np.testing.assert_array_equal(got[..., rot:], x[..., rot:])
  assert np.isclose((got ** 2).sum(), (x ** 2).sum())
  z = NR.apply_rope_f64(x, NR.rope_angles_f64(np.zeros((7, 3)), dims, 1e4),
                        mode)
  np.testing.assert_allclose(z, x, atol=0)


def test_rope_h3_table_form():
  """H3's own construction (cat per-axis freqs, cat with itself, rotate_half
  via cat(-x2, x1)) built here from its description gives the oracle's value."""
  pos = RNG.integers(0, 60, size=(9, 3))
  x = _rand(9, 128)
  inv = 1.0 / 10000.0 ** (np.arange(0, 32, 2) / 32)
  fr = pos[..., None] * inv[None, None]                    # (S, 3, 16)
  fr = np.concatenate([fr[:, 0], fr[:, 1], fr[:, 2]], -1)  # (S, 48)
  fr = np.concatenate([fr, fr], -1)                        # (S, 96)
  rotated, passed = x[:, :96], x[:, 96:]
  x1, x2 = rotated[:, :48], rotated[:, 48:]
  turned = np.concatenate([-x2, x1], -1)
  want = np.concatenate([rotated * np.cos(fr) + turned * np.sin(fr), passed],
                        -1)
  got = NR.apply_rope_f64(x, NR.rope_angles_f64(pos, (32, 32, 32), 1e4),
                          "half")
  np.testing.assert_allclose(got, want, atol=1e-12)


def test_rope_table_known_answer():
  """Hand-computed: rotate-half over 4 channels, pair 0 = (0, 2) by 90
  degrees, pair 1 = (1, 3) by 0; interleaved: pair 0 = (0, 1) by 90."""
  x = np.array([1.0, 2.0, 3.0, 4.0])[None, None, None]
  cos, sin = np.array([[0.0, 1.0]]), np.array([[1.0, 0.0]])
  got = NR.apply_rope_table_f64(x, cos, sin, "half")
  np.testing.assert_array_equal(got[0, 0, 0], [-3.0, 2.0, 1.0, 4.0])
  got = NR.apply_rope_table_f64(x, cos, sin, "pair")
  np.testing.assert_array_equal(got[0, 0, 0], [-2.0, 1.0, 3.0, 4.0])


@pytest.mark.parametrize("mode,dims", [("half", (44, 42, 42)),
                                       ("pair", (16, 56, 56)),
                                       ("half", (32, 32, 32))])
def test_rope_table_equals_positions(mode, dims):
  """cos/sin of the positional angles as a table give the positional path."""
  pos = RNG.integers(-5, 60, size=(11, 3))
  x = _rand(2, 11, 3, 128)
  ang = NR.rope_angles_f64(pos, dims, 1e4)
  got = NR.apply_rope_table_f64(x, np.cos(ang), np.sin(ang), mode)
  want = np.swapaxes(NR.apply_rope_f64(np.swapaxes(x, 1, 2), ang, mode), 1, 2)
  np.testing.assert_allclose(got, want, atol=1e-12)


def test_rope_table_reference_conventions():
  """H3's apply_rope with repeated-half (S, rotary) tables and MOSS's
  _rotate with (B, S, D) [sin | cos] rows both equal the table oracle on the
  mapping the kernel's Python layer uses (first half of H3's tables; MOSS
  cos = rows[D/2:], sin = rows[:D/2]); tables are arbitrary (not unit
  circle) so a swapped cos/sin or a dropped term shows."""
  x = _rand(2, 9, 3, 128)
  c, s = _rand(9, 48), _rand(9, 48)
  got = NR.h3_apply_rope_f64(x, np.concatenate([c, c], -1),
                             np.concatenate([s, s], -1))
  np.testing.assert_allclose(got, NR.apply_rope_table_f64(x, c, s, "half"),
                             atol=1e-12)
  rows = _rand(2, 9, 128)
  got = NR.moss_rotate_f64(x, rows)
  want = NR.apply_rope_table_f64(x, rows[..., 64:], rows[..., :64], "half")
  np.testing.assert_allclose(got, want, atol=1e-12)
  # per-batch tables differ per batch
  assert not np.allclose(got[0], NR.apply_rope_table_f64(
      x[:1], rows[1, :, 64:], rows[1, :, :64], "half")[0])


def test_rope_relative_position():
  """<rope(q, p), rope(k, p')> depends on p - p' only (1D)."""
  q, k = _rand(1, 64), _rand(1, 64)
  def dot(p1, p2):
    a = NR.apply_rope_f64(q, NR.rope_angles_f64(np.array([[p1, 0, 0]]),
                                                (64, 0, 0), 1e4), "half")
    b = NR.apply_rope_f64(k, NR.rope_angles_f64(np.array([[p2, 0, 0]]),
                                                (64, 0, 0), 1e4), "half")
    return float((a * b).sum())
  assert np.isclose(dot(3, 10), dot(20, 27))
  assert not np.isclose(dot(3, 10), dot(10, 3))


def test_qk_norm_rope_composition():
  x = _rand(2, 6, 3, 64)
  w = 1 + 0.02 * _rand(64)
  pos = RNG.integers(0, 50, size=(6, 3))
  hs = np.array([0.5, 1.0, 1.5])
  got = NR.qk_norm_rope_f64(x, w, 1e-6, pos, (64, 0, 0), 1e4, "half",
                            head_scale=hs, valid_len=4)
  assert np.all(got[:, 4:] == 0)
  y = torch.nn.functional.rms_norm(torch.from_numpy(x), (64,),
                                   torch.from_numpy(w), eps=1e-6).numpy()
  ang = NR.rope_angles_f64(pos, (64, 0, 0), 1e4)
  want = _as_complex_rotation(np.swapaxes(y, 1, 2), ang, "half")
  want = np.swapaxes(want, 1, 2) * hs[None, None, :, None]
  np.testing.assert_allclose(got[:, :4], want[:, :4], atol=1e-12)


# ------------------------------------------------------------------- fixed-m
def test_fixed_m_bound_is_cauchy_schwarz():
  q, k = _rand(2, 3, 17, 8), _rand(2, 3, 23, 8)
  mk = FM.fixed_m_operands(q, k, gate=5.0)
  for h in range(3):
    # brute force: the largest |logit| never exceeds the bound, and the bound
    # is attained for colinear maximal rows
    logits = np.einsum("bqd,bkd->bqk", q[:, h], k[:, h])
    qn = max(np.linalg.norm(q[b, h, i]) for b in range(2) for i in range(17))
    kn = max(np.linalg.norm(k[b, h, j]) for b in range(2) for j in range(23))
    assert np.abs(logits).max() <= qn * kn + 1e-12
    assert mk[0, h] == math.ceil(qn * kn)
    assert mk[1, h] == float(qn * kn <= 5.0)
  qq = np.zeros((1, 1, 2, 4)); qq[0, 0, 0] = [3, 0, 0, 4]
  kk = np.zeros((1, 1, 2, 4)); kk[0, 0, 1] = [0, 2, 0, 0]
  np.testing.assert_array_equal(FM.fixed_m_operands(qq, kk), [[10.0], [1.0]])


# ------------------------------------------------------------------- E4M3
def test_bf16_round_matches_torch_and_known_answers():
  """Hand-derived ties (1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties to
  even -> 1; 1 + 3*2^-8 -> 1 + 2^-6) and torch's float32 -> bfloat16 cast on
  random values."""
  assert FM.bf16_round(1.0 + 2.0**-8) == 1.0
  assert FM.bf16_round(1.0 + 3 * 2.0**-8) == 1.0 + 2.0**-6
  assert FM.bf16_round(-(1.0 + 2.0**-8 + 2.0**-20)) == -(1.0 + 2.0**-7)
  x = (RNG.standard_normal(20000) * 10.0 ** RNG.uniform(-6, 6, 20000))
  want = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).double()
  np.testing.assert_array_equal(FM.bf16_round(x), want.numpy())


def test_smooth_keys_invariants():
  """Smoothed keys: the real rows' mean is zero up to bf16 rounding, padded
  rows are zero, ks + mean reproduces k to bf16 rounding, and softmax
  attention is unchanged (a per-head key shift cancels)."""
  k = FM.bf16_round(RNG.standard_normal((2, 3, 50, 16)) + 2.0)
  ks, mean = FM.smooth_keys(k, kv_len=41)
  assert np.all(ks[:, :, 41:] == 0)
  assert np.abs(ks[:, :, :41].mean(axis=2)).max() < 0.02
  assert np.abs(ks[:, :, :41] + mean - k[:, :, :41]).max() <= 2.0**-6
  assert np.all(FM.bf16_round(ks) == ks)
  q = RNG.standard_normal((2, 3, 7, 16))
  v = RNG.standard_normal((2, 3, 50, 16))
  a = A.attention_f64(q, k, v, kv_len=41)
  b = A.attention_f64(q, ks + 0.0, v, kv_len=41)
  np.testing.assert_allclose(a, b, atol=2e-2)


def test_e4m3_known_answers():
  """Hand-derived codes: bias 7, 3 mantissa bits, max 448 = 0x7E."""
  x = [1.0, 448.0, 500.0, -1e6, 2.0**-9, 2.0**-10, 3 * 2.0**-10, 1.0625,
       1.1875, -2.0, 0.5, 0.0, -0.0, 240.0, 2.0**-6, 7 * 2.0**-9]
  want = [0x38, 0x7E, 0x7E, 0xFE, 0x01, 0x00, 0x02, 0x38,
          0x3A, 0xC0, 0x30, 0x00, 0x80, 0x77, 0x08, 0x07]
  assert P8.quantize_e4m3(x).tolist() == want
  assert P8.decode_e4m3(0x7E) == 448.0 and np.isnan(P8.decode_e4m3(0x7F))


def test_e4m3_matches_torch_cast_and_round_trips():
  """Every finite code decodes and re-encodes to itself; random values agree
  with torch's float8_e4m3fn cast after the 448 clamp."""
  codes = np.array([c for c in range(256) if c & 0x7F != 0x7F])
  np.testing.assert_array_equal(P8.quantize_e4m3(P8.decode_e4m3(codes)),
                                codes)
  rng = np.random.default_rng(7)
  x = np.concatenate([rng.standard_normal(20000) * 50,
                      rng.standard_normal(2000) * 1e-2,
                      np.ldexp(rng.integers(1, 16, 500) / 2.0, -10)])
  t = torch.clamp(torch.tensor(x, dtype=torch.float32), -448, 448)
  ref = t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
  np.testing.assert_array_equal(P8.quantize_e4m3(x.astype(np.float32)), ref)


# ------------------------------------------------------------ block-sparse
def test_masked_attention_oracle():
  """Full mask = dense; a block mask = dense attention over the gathered
  keys of each query block; an all-false row is zero."""
  q, k, v = _rand(1, 2, 40, 8), _rand(1, 2, 30, 8), _rand(1, 2, 30, 8)
  full = np.ones((40, 30), bool)
  np.testing.assert_allclose(SP.attention_masked_f64(q, k, v, full),
                             A.attention_f64(q, k, v), atol=1e-12)
  table = [[0, 2], [1]]            # block_q 20, block_kv 10
  mask = SP.block_mask(40, 30, 20, 10, table)
  got = SP.attention_masked_f64(q, k, v, mask)
  keys0 = np.r_[0:10, 20:30]
  np.testing.assert_allclose(
      got[:, :, :20], A.attention_f64(q[:, :, :20], k[:, :, keys0],
                                      v[:, :, keys0]), atol=1e-12)
  np.testing.assert_allclose(
      got[:, :, 20:], A.attention_f64(q[:, :, 20:], k[:, :, 10:20],
                                      v[:, :, 10:20]), atol=1e-12)
  mask[5] = False
  assert (SP.attention_masked_f64(q, k, v, mask)[:, :, 5] == 0).all()


@pytest.mark.parametrize("args", [
    (200, 40, 16, 1, 32, 32), (200, 0, 10, 2, 64, 16), (150, 60, 7, 0, 16, 48),
    (97, 97, 5, 3, 32, 32)])
def test_window_table_matches_bruteforce(args):
  from diffusers_tpu_amd.kernels.sparse_splash import temporal_window_table
  assert temporal_window_table(*args) == SP.window_table_bruteforce(*args)
