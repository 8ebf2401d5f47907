"""Host-side conversion of the reference's block-sparse tables
(kernels/sparse_splash.py:439-462) into the kernel's 256-row / 64-key units,
checked against the oracle's key mask; runs on the CPU."""
import numpy as np
import pytest

from diffusers_tpu_amd.kernels import sparse_splash as S
from oracle import sparse as SP


def _mask_of(tt, hq, sq, skv):
  span, ids = tt.span.numpy(), tt.ids.numpy()
  mask = np.zeros((hq, sq, skv), bool)
  for h in range(hq):
    for i in range(span.shape[1]):
      for t in ids[span[h, i, 0]:span[h, i, 1]]:
        mask[h, i * 256:(i + 1) * 256, t * 64:(t + 1) * 64] = True
  return mask


@pytest.mark.parametrize("sq,skv,bq,bkv,kv_len", [
    (1000, 1000, 256, 64, None), (1000, 900, 512, 128, 801),
    (300, 700, 2048, 2048, 650), (2048, 2048, 1024, 192, None)])
def test_tile_table_equals_block_mask(sq, skv, bq, bkv, kv_len):
  rng = np.random.default_rng(sq + skv)
  nq, nk = -(-sq // min(bq, sq)), -(-skv // min(bkv, skv))
  table = [sorted(rng.choice(nk, size=rng.integers(1, nk + 1), replace=False)
                  .tolist()) for _ in range(nq)]
  # every row keeps block 0 so no row is empty below kv_len
  table = [sorted(set(r) | {0}) for r in table]
  tt = S.build_tile_table(table, sq=sq, skv=skv, heads=2, block_q=bq,
                          block_kv=bkv, kv_len=kv_len, device="cpu")
  want = SP.block_mask(sq, skv, bq, bkv, table)
  if kv_len is not None:
    want[:, kv_len:] = False
  got = _mask_of(tt, 2, sq, skv)
  # the kernel masks keys >= kv_len inside a tile itself
  if kv_len is not None:
    got[:, :, kv_len:] = False
  assert (got == want[None]).all()


def test_head_classes_and_dyn_form():
  tbl0 = [[0], [1], [0, 1]]            # block_q = block_kv = 256, S = 600
  tbl1 = [[0, 1, 2]] * 3
  tt = S.build_tile_table(([tbl0, tbl1], [1, 0, 1]), sq=600, skv=600,
                          heads=3, block_q=256, block_kv=256, device="cpu")
  m = _mask_of(tt, 3, 600, 600)
  assert (m[0] == SP.block_mask(600, 600, 256, 256, tbl1)).all()
  assert (m[1] == SP.block_mask(600, 600, 256, 256, tbl0)).all()
  table = np.array([[[0, 0], [1, 1], [0, 1]]])
  counts = np.array([[1, 1, 2]])
  assert S._dyn_table((table, counts)) == tbl0


def test_rejects_unaligned_blocks_and_empty_rows():
  with pytest.raises(NotImplementedError):
    S.build_tile_table([[0]] * 8, sq=1024, skv=1024, heads=1, block_q=128,
                       block_kv=128, device="cpu")
  with pytest.raises(NotImplementedError):
    S.build_tile_table([[0]] * 4, sq=1024, skv=1024, heads=1, block_q=256,
                       block_kv=96, device="cpu")
  with pytest.raises(ValueError):      # row 1 only sees keys past kv_len
    S.build_tile_table([[0], [3]], sq=512, skv=512, heads=1, block_q=256,
                       block_kv=128, kv_len=300, device="cpu")
