"""Packed V (dt_pack_v, dt_flash_fwd_ex with vt): the layout against its
definition in include/dt_attention.h, and attention from packed V against
the row-major entry points.  The packed path feeds the same operands to the
same MFMAs in the same order, so its results must be bit-identical."""
import numpy as np
import pytest
import torch

from gpu_helpers import banner, seeded

pytestmark = pytest.mark.gpu

PERM = [(j & 3) | ((j & 4) << 1) | ((j & 8) >> 1) for j in range(16)]


@pytest.fixture(scope="module")
def sp():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.kernels import splash
  return splash


def _expected_layout(v, kv_end, tiles):
  """[B*Hkv, tiles, 128, 64]: column 16g + j of tile t holds key
  64t + 16g + PERM[j]; zero from kv_end."""
  b, h, s, d = v.shape
  want = np.zeros((b * h, tiles, d, 64), np.uint16)
  vv = v.view(torch.int16).cpu().numpy().astype(np.uint16).reshape(b * h, s, d)
  for t in range(tiles):
    for col in range(64):
      key = 64 * t + 16 * (col // 16) + PERM[col % 16]
      if key < kv_end:
        want[:, t, :, col] = vv[:, key, :]
  return want


@pytest.mark.parametrize("shape,kv_len", [((1, 2, 300, 128), None),
                                          ((2, 3, 200, 128), 131),
                                          ((1, 1, 64, 128), None)])
def test_pack_layout(sp, shape, kv_len):
  banner(f"pack_v layout {shape} kv_len={kv_len}")
  v = seeded(shape, 170)
  vt, tiles = sp.pack_v(v, kv_len)
  torch.cuda.synchronize()
  kv_end = kv_len or shape[2]
  assert tiles == (kv_end + 63) // 64
  got = vt.view(torch.int16).cpu().numpy().astype(np.uint16)
  np.testing.assert_array_equal(got.reshape(-1, tiles, 128, 64),
                                _expected_layout(v, kv_end, tiles))


def test_pack_strided_view(sp):
  """V as a (B, H, S, D) view of (B, S, H, D) storage packs the same."""
  banner("pack_v strided")
  base = seeded((1, 250, 3, 128), 171)
  v = base.transpose(1, 2)
  a, _ = sp.pack_v(v)
  b, _ = sp.pack_v(v.contiguous())
  torch.cuda.synchronize()
  assert torch.equal(a, b)


CASES = [
    # (B, Hq, Hkv, Sq, Skv, kv_len)
    (1, 4, 4, 700, 1000, None),
    (2, 6, 2, 333, 900, 811),        # GQA, kv_len mid-tile
    (1, 2, 2, 1, 64, None),          # one query, one tile
]


@pytest.mark.parametrize("case", CASES)
def test_packed_equals_rowmajor(sp, case):
  b, hq, hkv, sq, skv, kv_len = case
  banner(f"packed vs row-major {case}")
  q = seeded((b, hq, sq, 128), 172)
  k = seeded((b, hkv, skv, 128), 173)
  v = seeded((b, hkv, skv, 128), 174)
  pv = sp.pack_v(v, kv_len)
  for qk8 in (False, True):
    a = sp._launch(q, k, v, None, kv_len, qk_fp8=qk8)
    c = sp._launch(q, k, v, None, kv_len, qk_fp8=qk8, packed_v=pv)
    ra = sp._launch(q, k, v, None, kv_len, residual=True, qk_fp8=qk8)
    rc = sp._launch(q, k, v, None, kv_len, residual=True, qk_fp8=qk8,
                    packed_v=pv)
    torch.cuda.synchronize()
    assert torch.equal(a, c), f"qk8={qk8}"
    for x, y in zip(ra, rc):
      assert torch.equal(x, y), f"residual qk8={qk8}"


def test_packed_blocksparse_equals_rowmajor(sp):
  from diffusers_tpu_amd import _lib
  from diffusers_tpu_amd.kernels import sparse_splash
  banner("packed vs row-major, block-sparse")
  q = seeded((1, 2, 1024, 128), 175)
  k = seeded((1, 2, 2048, 128), 176)
  v = seeded((1, 2, 2048, 128), 177)
  table = sparse_splash.temporal_window_table(2048, 256, 256, 1, 512, 256)
  tt = sparse_splash.build_tile_table(table[:2], sq=1024, skv=2048, heads=2,
                                      block_q=512, block_kv=256)
  want = sparse_splash.attention(q, k, v, scale=None, block_q=512,
                                 block_kv=256, kv_table=tt)
  got = sp._call_ex(q, k, 0, None, sp.pack_v(v), None, False, 2, 2048,
                    1 / 128 ** 0.5, 2048, None, tt.span, tt.ids)
  torch.cuda.synchronize()
  assert torch.equal(got, want)


def test_packed_errors(sp):
  from diffusers_tpu_amd import _lib
  banner("packed errors")
  v = seeded((1, 1, 100, 128), 178)
  vt = torch.empty(2 * 128 * 64, device="cuda", dtype=torch.bfloat16)
  lib = _lib.load()
  st = torch.cuda.current_stream().cuda_stream
  s = _lib.i64_array(*v.stride()[:3])
  # fewer tiles than 100 keys need
  assert lib.dt_pack_v(v.data_ptr(), vt.data_ptr(), 1, 1, 100, 128, s, 0, None, 1,
                       st) != 0
  assert "vt_tiles" in lib.dt_last_error().decode()
  assert lib.dt_pack_v(v.data_ptr(), vt.data_ptr(), 1, 1, 100, 64, s, 0, None, 2,
                       st) != 0
  with pytest.raises(ValueError):
    sp.pack_v(v, out=torch.empty(10, device="cuda", dtype=torch.bfloat16))


def test_attention_packed_and_split_large(sp):
  """attention() at a length that takes packed V (>= PACKED_V_MIN_KEYS) and a
  grid (2 heads x 157 query blocks) whose last round is split, against the
  float64 oracle on sampled rows, including the split blocks' rows."""
  from diffusers_tpu_amd import _lib
  from gpu_helpers import assert_attn_close, to64
  from oracle import attention as A
  banner("attention packed V + tail split, S=40000")
  b, h, s, n = 1, 2, 40000, 39001
  assert n >= sp.PACKED_V_MIN_KEYS
  assert _lib.load().dt_flash_fwd_workspace_bytes(b, h, s, s, n, 128) > 0
  q = seeded((b, h, s, 128), 179)
  k = seeded((b, h, s, 128), 180)
  v = seeded((b, h, s, 128), 181)
  got = sp.attention(q, k, v, scale=None, block_q=0, block_kv=0,
                     block_kv_compute=0, kv_len=n)
  torch.cuda.synchronize()
  rows = np.r_[0:5, 12345:12350, s - 300:s:37, s - 5:s]
  want = A.attention_rows_f64(to64(q), to64(k), to64(v), rows, kv_len=n)
  assert_attn_close(to64(got)[:, :, rows], want, "packed + split")
