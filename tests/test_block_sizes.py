"""Block-size resolution and launch plan (kernels/block_sizes.py): the
reference's entry points (kernels/block_sizes.py:442-640,
kernels/splash.py:529-563) answering for the gfx950 tile, and the plan
dt_flash_fwd_ex follows (GPU)."""
import pytest
import torch

from diffusers_tpu_amd.kernels import block_sizes as bs


def test_local_blocks_clamps_like_the_reference():
  # each block at most its extent
  assert bs.local_blocks(100, 5000, 256, 64, 64) == (100, 64, 64)
  assert bs.local_blocks(4096, 40, 256, 64, 64) == (256, 40, 40)
  # a clamped K/V block the compute block does not divide: one step
  assert bs.local_blocks(4096, 300, 2048, 2048, 256) == (2048, 300, 300)
  assert bs.local_blocks(4096, 512, 2048, 2048, 256) == (2048, 512, 256)
  with pytest.raises(ValueError):
    bs.local_blocks(0, 10, 256, 64, 64)
  with pytest.raises(ValueError):
    bs.local_blocks(10, 10, 256, -1, 64)


def test_resolution_order_pinned_tuned_default():
  spec = bs.MI355X_SPEC
  assert bs.resolve_block_sizes(350784, 350784, 128, {}, "online", spec) == {
      "block_q": 256, "block_kv": 64, "block_kv_compute": 64}
  # a pinned field wins, the others stay tuned
  got = bs.resolve_block_sizes(4608, 4608, 128, {"block_q": 2048,
                                                 "block_kv": None},
                               "residual-fixedm", spec)
  assert got == {"block_q": 2048, "block_kv": 64, "block_kv_compute": 64}
  # short sequences: the tile clamps to the extents
  assert bs.resolve_block_sizes(40, 30, 64, {}, "online", spec) == {
      "block_q": 40, "block_kv": 30, "block_kv_compute": 30}
  assert bs.ring_step_blocks(8192, 128, spec=spec, use_fixed_m=True) == \
      bs.DEFAULT_BLOCKS
  assert bs.ring_step_blocks(8192, 128, spec=spec,
                             pinned={"block_kv": 512})["block_kv"] == 512
  assert bs.rank_block_candidates(48872) == [bs.DEFAULT_BLOCKS]
  with pytest.raises(NotImplementedError):
    bs.autotune_block_sizes(4096, head_dim=100)
  with pytest.raises(ValueError):
    bs.rank_block_candidates(4096, top_k=0)


def test_spec_fallback_without_gpu():
  if torch.cuda.is_available():
    spec = bs.detect_spec()
    assert spec.compute_units == torch.cuda.get_device_properties(
        torch.cuda.current_device()).multi_processor_count
  else:
    assert bs.detect_spec() == bs.MI355X_SPEC
  assert bs.MI355X_SPEC.compute_units == 256 and bs.MI355X_SPEC.xcds == 8
  assert bs.MI355X_SPEC.lds_bytes == 160 * 1024


@pytest.mark.gpu
def test_launch_plan_matches_the_planner():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd import _lib
  lib = _lib.load()
  n_cu = torch.cuda.get_device_properties(0).multi_processor_count
  unit = 256 * 130 * 4
  # a full last round: nothing to split
  p = bs.launch_plan(1, n_cu, 256, 8192)
  assert (p.query_blocks, p.split_parts, p.tail_blocks, p.workspace_bytes) \
      == (n_cu, 1, 0, 0)
  assert p.whole_blocks == n_cu and p.key_tiles == 128 and p.rounds == 1.0
  # one block of 128 tiles: 10 parts, the bytes dt_flash_fwd_ex can use
  p = bs.launch_plan(1, 1, 256, 8192)
  assert (p.split_parts, p.tail_blocks, p.whole_blocks) == (10, 1, 0)
  assert p.workspace_bytes == 10 * unit == lib.dt_flash_fwd_workspace_bytes(
      1, 1, 256, 8192, 0, 128)
  # a smaller workspace: the best split that fits, or none
  assert bs.launch_plan(1, 1, 256, 8192, workspace_bytes=4 * unit).split_parts \
      == 4
  p = bs.launch_plan(1, 1, 256, 8192, workspace_bytes=0)
  assert (p.split_parts, p.workspace_bytes, p.whole_blocks) == (1, 0, 1)
  # head dims plan as the kernel's: 96 as 128, 40 as 64
  assert bs.launch_plan(1, 1, 256, 8192, head_dim=96) == \
      bs.launch_plan(1, 1, 256, 8192)
  assert bs.launch_plan(1, 1, 256, 8192, head_dim=40).workspace_bytes == \
      10 * 256 * 66 * 4
  with pytest.raises(NotImplementedError):
    bs.launch_plan(1, 1, 256, 8192, head_dim=264)
  with pytest.raises(NotImplementedError):
    bs.launch_plan(1, 1, 256, 8192, head_dim=192, qk_fp8=True)
  wide = bs.launch_plan(1, 1, 256, 8192, head_dim=192)  # runs as 256
  assert (wide.split_parts, wide.workspace_bytes, wide.query_blocks,
          wide.key_tiles) == (1, 0, 2, 256)
  if n_cu == 256:
    # I1: 864 blocks of 69 tiles, the last 96 in 2 parts each
    p = bs.launch_plan(2, 24, 4608, kv_len=4396)
    assert (p.query_blocks, p.key_tiles, p.split_parts, p.tail_blocks,
            p.whole_blocks) == (864, 69, 2, 96, 768)
    # V7: 6855 blocks, the last 199 in 9 parts
    p = bs.launch_plan(1, 5, 350784)
    assert (p.query_blocks, p.split_parts, p.tail_blocks) == (6855, 9, 199)


def test_splash_block_sizes_record():
  """``splash.BlockSizes`` keeps the reference's record: three slots,
  ``block_kv_compute`` defaulting to ``block_kv`` (kernels/splash.py:92-112)."""
  from diffusers_tpu_amd.kernels import splash, sparse_splash
  b = splash.BlockSizes(2048, 1024)
  assert (b.block_q, b.block_kv, b.block_kv_compute) == (2048, 1024, 1024)
  assert splash.BlockSizes(1, 2, 3).block_kv_compute == 3
  assert sparse_splash.BlockSizes is splash.BlockSizes
  with pytest.raises(AttributeError):
    b.other = 1
