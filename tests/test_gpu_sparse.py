"""Block-sparse attention on the GPU (kernels/sparse_splash.py) against the
float64 masked-softmax oracle; a full table must reproduce the dense kernel
bit for bit (kernels/sparse_splash.py:1-5)."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A
from oracle import fp8 as P8
from oracle import sparse as SP

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sp():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.kernels import sparse_splash
  return sparse_splash


def test_full_table_is_bit_identical_to_dense(sp):
  """Through the C ABI without a workspace, so both run the classic grid
  with no split: a table listing every key tile gives the dense result bit
  for bit (the Python entry points may schedule the two differently)."""
  from diffusers_tpu_amd import _lib
  banner("sparse full table vs dense")
  q = seeded((2, 3, 700, 128), 120)
  k = seeded((2, 3, 900, 128), 121)
  v = seeded((2, 3, 900, 128), 122)
  tt = sp.build_tile_table([list(range(2))] * 2, sq=700, skv=900,
                           heads=3, block_q=512, block_kv=512, kv_len=811)
  lib = _lib.load()
  s3 = lambda t: _lib.i64_array(*t.stride()[:3])
  st = torch.cuda.current_stream().cuda_stream
  a = torch.empty_like(q)
  b = torch.empty_like(q)
  scale = 1 / 128 ** 0.5
  _lib.check("dt_flash_fwd_blocksparse", lib.dt_flash_fwd_blocksparse(
      q.data_ptr(), k.data_ptr(), 0, v.data_ptr(), a.data_ptr(), 2, 3, 3, 700,
      900, 128, s3(q), s3(k), s3(v), s3(a), scale, 811, None,
      tt.span.data_ptr(), tt.ids.data_ptr(), None, None, None, st))
  _lib.check("dt_flash_fwd", lib.dt_flash_fwd(
      q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(), 2, 3, 3, 700,
      900, 128, s3(q), s3(k), s3(v), s3(b), scale, 811, None, None, None,
      None, st))
  torch.cuda.synchronize()
  assert torch.equal(a, b)
  # and the Python entry points agree to bf16 rounding
  c = sp.attention(q, k, v, scale=None, block_q=512, block_kv=512,
                   block_kv_compute=512, kv_len=811)
  import diffusers_tpu_amd as dta
  d = dta.attention(q, k, v, scale=None, block_q=512, block_kv=512,
                    block_kv_compute=512, kv_len=811)
  torch.cuda.synchronize()
  assert (c.float() - d.float()).abs().max().item() <= 2 ** -7


@pytest.mark.parametrize("case", [
    # (seq, video_start, rows_per_frame, window, block_q, block_kv, kv_len)
    (3000, 512, 256, 1, 512, 256, None),
    (2600, 300, 128, 2, 256, 128, 2411),
    (1536, 0, 64, 1, 256, 64, None),
])
def test_temporal_window_matches_oracle(sp, case):
  seq, vs, rpf, win, bq, bkv, kv_len = case
  banner(f"sparse temporal window {case}")
  q = seeded((1, 2, seq, 128), 123)
  k = seeded((1, 2, seq, 128), 124)
  v = seeded((1, 2, seq, 128), 125)
  table = sp.temporal_window_table(seq, vs, rpf, win, bq, bkv)
  got = sp.attention(q, k, v, scale=None, block_q=bq, block_kv=bkv,
                     block_kv_compute=bkv, kv_table=table, kv_len=kv_len)
  torch.cuda.synchronize()
  mask = SP.block_mask(seq, seq, bq, bkv, table)
  if kv_len is not None:
    mask[:, kv_len:] = False
  want = SP.attention_masked_f64(to64(q), to64(k), to64(v), mask)
  assert_attn_close(to64(got), want, f"window {case}")
  assert not mask.all(), "the case must actually skip blocks"


def test_head_classes_qk_fp8_and_tile_table_reuse(sp):
  banner("sparse head classes, qk_fp8, TileTable reuse")
  seq = 1024
  q = seeded((1, 4, seq, 128), 126)
  k = seeded((1, 2, seq, 128), 127)      # GQA 2:1
  v = seeded((1, 2, seq, 128), 128)
  narrow = sp.temporal_window_table(seq, 256, 128, 1, 256, 256)
  wide = sp.temporal_window_table(seq, 256, 128, 3, 256, 256)
  heads = [0, 1, 1, 0]
  tt = sp.build_tile_table(([narrow, wide], heads), sq=seq, skv=seq, heads=4,
                           block_q=256, block_kv=256)
  mask = np.stack([SP.block_mask(seq, seq, 256, 256, [narrow, wide][c])
                   for c in heads])
  got = sp.attention(q, k, v, scale=None, block_q=256, block_kv=256,
                     kv_table=tt)
  want = SP.attention_masked_f64(to64(q), to64(k), to64(v), mask)
  assert_attn_close(to64(got), want, "head classes")
  got8 = sp.attention(q, k, v, scale=None, block_q=256, block_kv=256,
                      kv_table=tt, qk_fp8=True)
  c = np.log2(np.e) / np.sqrt(128)
  q8 = P8.e4m3_round(to64((q.float() * c).to(torch.bfloat16)))
  k8 = P8.e4m3_round(to64(k))
  want8 = SP.attention_masked_f64(q8, k8, to64(v), mask, scale=np.log(2.0))
  assert_attn_close(to64(got8), want8, "head classes qk_fp8")


def test_residual_and_fixed_m(sp):
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  from diffusers_tpu_amd.kernels.splash import merge_residuals
  banner("sparse residual + fixed-m")
  seq = 1280
  q = seeded((1, 2, seq, 128), 129)
  k = seeded((1, 2, seq, 128), 130)
  k = (k.float() - k.float().mean(dim=2, keepdim=True)).to(k.dtype)
  v = seeded((1, 2, seq, 128), 131)
  table = sp.temporal_window_table(seq, 256, 256, 1, 256, 256)
  mk = fmb.fixed_m_operands_from_norms(fmb.fixed_m_query_norms(q),
                                       fmb.max_row_norm_per_head(k))
  o, m, l = sp.residual_attention(q, k, v, scale=None, block_q=256,
                                  block_kv=256, kv_table=table,
                                  use_fixed_m=True, mk=mk)
  mask = SP.block_mask(seq, seq, 256, 256, table)
  want = SP.attention_masked_f64(to64(q), to64(k), to64(v), mask)
  assert_attn_close(to64(o) / to64(l), want, "sparse residual fixed-m")
  assert (to64(m)[0, :, :, 0] == (to64(mk[0]) - 88.0)[:, None]).all()


def test_empty_row_comes_out_zero(sp):
  banner("sparse empty table row")
  q = seeded((1, 1, 512, 128), 132)
  k = seeded((1, 1, 512, 128), 133)
  v = seeded((1, 1, 512, 128), 134)
  tt = sp.build_tile_table([[0]], sq=512, skv=512, heads=1, block_q=512,
                           block_kv=512)
  # hand-edit: query block 1 gets an empty span
  tt.span[0, 1, 0] = tt.span[0, 1, 1]
  got = sp.attention(q, k, v, scale=None, block_q=512, block_kv=512,
                     kv_table=tt)
  torch.cuda.synchronize()
  assert (got[0, 0, 256:] == 0).all()
  mask = np.zeros((512, 512), bool)
  mask[:256] = True
  want = SP.attention_masked_f64(to64(q), to64(k), to64(v), mask)
  assert_attn_close(to64(got), want, "empty row")


def test_sparse_head_dim_96(sp):
  banner("sparse head_dim 96")
  seq = 1000
  q = seeded((1, 2, seq, 96), 135)
  k = seeded((1, 2, seq, 96), 136)
  v = seeded((1, 2, seq, 96), 137)
  table = sp.temporal_window_table(seq, 256, 128, 1, 256, 256)
  got = sp.attention(q, k, v, scale=None, block_q=256, block_kv=256,
                     kv_table=table)
  assert got.shape == q.shape
  mask = SP.block_mask(seq, seq, 256, 256, table)
  want = SP.attention_masked_f64(to64(q), to64(k), to64(v), mask)
  assert_attn_close(to64(got), want, "sparse d=96")
