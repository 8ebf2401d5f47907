"""Tail split (dt_flash_fwd_ex with a workspace): the query blocks of a
partly filled last round of workgroups run as 2-8 key-range parts whose
(o, m, l) are merged in LSE space (kernels/splash.py:653-662).  Checked
against the unsplit kernel (no workspace) and the float64 oracle, in the
normalized and the residual form."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sp():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.kernels import splash
  return splash


def _cus():
  return torch.cuda.get_device_properties(0).multi_processor_count


def _nosplit(sp, q, k, v, kv_len, residual, mk=None, k_format=0):
  """dt_flash_fwd_ex without a workspace (no split)."""
  from diffusers_tpu_amd import _lib
  b, hq, sq, d = q.shape
  _, hkv, skv, _ = k.shape
  s3 = lambda t: _lib.i64_array(*t.stride()[:3])
  st = torch.cuda.current_stream().cuda_stream
  n = kv_len or skv
  if residual:
    o32 = torch.empty((b, hq, sq, d), device="cuda", dtype=torch.float32)
    m = torch.empty((b, hq, sq, 1), device="cuda", dtype=torch.float32)
    l = torch.empty_like(m)
    outs = (None, None, o32.data_ptr(), m.data_ptr(), l.data_ptr())
  else:
    o = torch.empty_like(q)
    outs = (o.data_ptr(), s3(o), None, None, None)
  rc = _lib.load().dt_flash_fwd_ex(
      q.data_ptr(), k.data_ptr(), k_format, v.data_ptr(), s3(v), None, 0,
      outs[0], b, hq, hkv, sq, skv, d, s3(q), s3(k), outs[1], 1 / d ** 0.5, n,
      None, None if mk is None else mk.data_ptr(), None, None, *outs[2:], None, 0,
      st)
  _lib.check("dt_flash_fwd_ex", rc)
  return (o32, m, l) if residual else o


def test_plan_sizes(sp):
  from diffusers_tpu_amd import _lib
  lib = _lib.load()
  ws = lambda *a: lib.dt_flash_fwd_workspace_bytes(*a)
  n_cu = _cus()
  banner(f"split plan, {n_cu} CUs")
  unit = 256 * 130 * 4          # one part's rows: o (128 floats), m, l
  # a full last round: no split
  assert ws(1, n_cu, 256, 8192, 0, 128) == 0
  # one query block of 128 key tiles: 10 parts (13 tiles + 8 of start-up
  # each + 10 for the merge = 31, against 136 unsplit; 16 parts: 32)
  assert ws(1, 1, 256, 8192, 0, 128) == 10 * unit
  # too few key tiles to split (2 tiles -> at most one part)
  assert ws(1, 1, 256, 128, 0, 128) == 0
  # head dim 64: rows of 64 floats
  assert ws(1, 1, 256, 8192, 0, 64) == 10 * 256 * 66 * 4
  assert ws(1, 1, 256, 8192, 0, 96) == 0
  if n_cu == 256:
    # P (B1 H8 S1024 D64, 32 blocks of 16 tiles): 4 parts (4 + 8 + 4 = 16;
    # 8 parts: 18)
    assert ws(1, 8, 1024, 1024, 0, 64) == 32 * 4 * 256 * 66 * 4
    # V7: the last 199 of 6855 blocks, 9 parts each (7 rounds of 609 + 8
    # tiles, against 5489 unsplit)
    assert ws(1, 5, 350784, 350784, 0, 128) == 199 * 9 * unit
    # I1: the last 96 of 864 blocks, 2 parts each (5 would be 2 rounds of
    # 14 + 8 tiles, against one of 35 + 8)
    assert ws(2, 24, 4608, 4608, 4396, 128) == 96 * 2 * unit


CASES = [
    # (B, Hq, Hkv, Sq, Skv, kv_len[, D])
    (2, 4, 2, 700, 3000, 2901, 64),   # head dim 64
    (1, 2, 2, 300, 4096, None),       # 4 blocks -> 8 parts each
    (2, 4, 2, 700, 3000, 2901),       # GQA, kv_len mid-tile
    (1, 3, 3, 256, 520, None),        # few tiles: ragged part sizes
]


@pytest.mark.parametrize("case", CASES)
def test_split_matches_unsplit_and_oracle(sp, case):
  b, hq, hkv, sq, skv, kv_len = case[:6]
  d = case[6] if len(case) > 6 else 128
  banner(f"split {case}")
  q = seeded((b, hq, sq, d), 180)
  k = seeded((b, hkv, skv, d), 181)
  v = seeded((b, hkv, skv, d), 182)
  from diffusers_tpu_amd import _lib
  assert _lib.load().dt_flash_fwd_workspace_bytes(b, hq, sq, skv, kv_len or 0,
                                                  d) > 0
  got = sp._launch(q, k, v, None, kv_len)
  ref = _nosplit(sp, q, k, v, kv_len, False)
  torch.cuda.synchronize()
  want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=kv_len)
  assert_attn_close(to64(got), want, "split vs oracle")
  assert (got.float() - ref.float()).abs().max().item() <= 2 ** -7
  # residual form: o/l equal, m within the kernel's bound of the row max
  o32, m, l = sp._launch(q, k, v, None, kv_len, residual=True)
  r32, rm, rl = _nosplit(sp, q, k, v, kv_len, True)
  torch.cuda.synchronize()
  wo, wm, wl = A.residual_f64(to64(q), to64(k), to64(v), kv_len=kv_len)
  assert_attn_close(to64(o32) / to64(l), wo / wl, "split residual o/l")
  # each part rounds its probabilities to bf16 against its own reference
  # m, so split and unsplit differ at bf16 rounding level, not fp32
  np.testing.assert_allclose(to64(o32) / to64(l), to64(r32) / to64(rl),
                             atol=1e-3, rtol=0)
  # m: within 2^13 of the row max, up to the shift bf16 rounding of c*q
  # moves a logit by (as tests/test_gpu_attention.py bounds it); the
  # m-invariant lse = m + log2(l) as the unsplit kernel's
  c = np.log2(np.e) / np.sqrt(float(d))
  n = kv_len or skv
  kr = np.repeat(to64(k)[:, :, :n], hq // hkv, axis=1)
  shift = 2.0**-9 * np.einsum("bhid,bhjd->bhij", np.abs(c * to64(q)),
                              np.abs(kr)).max(-1)[..., None]
  gm = to64(m)
  assert (gm <= wm + shift + 1e-4).all() and (gm >= wm - 13 - shift).all()
  lse = gm + np.log2(to64(l))
  np.testing.assert_allclose(lse, to64(rm) + np.log2(to64(rl)), atol=3e-3,
                             rtol=0)


def test_split_qk8_fixed_m_and_sparse(sp):
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb, sparse_splash
  banner("split qk8 / fixed-m / sparse")
  q = seeded((1, 2, 512, 128), 183)
  k = seeded((1, 2, 4096, 128), 184)
  k = (k.float() - k.float().mean(dim=2, keepdim=True)).to(torch.bfloat16)
  v = seeded((1, 2, 4096, 128), 185)
  want = A.attention_f64(to64(q), to64(k), to64(v))
  # fixed-m through the split: every part starts from the same m
  mk = fmb.fixed_m_operands(q.float() * (1.4426950408889634 / 128 ** 0.5), k,
                            gate=fmb.FIXED_M_SAFE_BOUND)
  got = sp._launch(q, k, v, None, None, mk=mk)
  o32, m, l = sp._launch(q, k, v, None, None, residual=True, mk=mk)
  torch.cuda.synchronize()
  assert_attn_close(to64(got), want, "split fixed-m")
  fixed = to64(mk[0]) - 88.0
  assert (to64(m)[0, :, :, 0] == fixed[:, None]).all()
  # qk8 split vs qk8 unsplit
  got8 = sp._launch(q, k, v, None, None, qk_fp8=True)
  from diffusers_tpu_amd.kernels.fp8_cast import quantize_saturating
  ref8 = _nosplit(sp, q, quantize_saturating(k), v, None, False, k_format=1)
  torch.cuda.synchronize()
  assert (got8.float() - ref8.float()).abs().max().item() <= 2 ** -7
  # block-sparse: rows whose tile list is shorter than the part count leave
  # some parts empty; the merge skips them
  from oracle import sparse as SP
  for table in ([[0, 5, 9], [1]], [[0], list(range(0, 64, 3))]):
    tt = sparse_splash.build_tile_table(table, sq=512, skv=4096, heads=2,
                                        block_q=256, block_kv=64)
    gs = sparse_splash.attention(q, k, v, scale=None, block_q=256,
                                 block_kv=64, kv_table=tt)
    torch.cuda.synchronize()
    mask = SP.block_mask(512, 4096, 256, 64, table)
    ws = SP.attention_masked_f64(to64(q), to64(k), to64(v), mask)
    assert_attn_close(to64(gs), ws, f"split sparse {table[0][:3]}")
