"""Block sizes and launch plan of the gfx950 attention kernel.

Counterpart of the reference's block-size resolution
(kernels/block_sizes.py:442-703) and of its per-call clamp
(kernels/splash.py:529-563).  The reference's Pallas kernel takes
``(block_q, block_kv, block_kv_compute)`` per call and tunes them per shape
from a VMEM / MXU cost model.  The gfx950 kernel's tile is fixed by its
mapping onto the hardware: 256 query rows per workgroup (8 wavefronts x 32
rows, one workgroup per CU, whose 128 KiB LDS ring of K/V stages it fills)
and 64 keys per stage.  What a shape decides here is the launch plan: how
the query blocks of a partly filled last round of workgroups are split
over their key tiles (``launch_plan``, from ``dt_flash_fwd_plan``, the
planner ``dt_flash_fwd_ex`` itself uses).

The reference's entry points keep their names, arguments and resolution
order (pinned, else tuned, else default), so callers that resolve blocks
before calling attention run unchanged; the blocks they get describe the
gfx950 tile, and ``attention`` accepts and ignores block arguments.
"""
from __future__ import annotations

import ctypes
import dataclasses
import logging
from typing import Mapping, NamedTuple

_logger = logging.getLogger(__name__)

ROWS_PER_WORKGROUP = 256  # query rows of one workgroup (8 wavefronts x 32)
KEYS_PER_TILE = 64        # keys of one LDS stage


@dataclasses.dataclass(frozen=True)
class GpuSpec:
  """Device parameters the plan depends on (the reference's ``TpuSpec``,
  kernels/block_sizes.py:144-170).

  Attributes:
    name: Device name.
    arch: Target the kernels are built for (``gfx950``).
    compute_units: CUs; one attention workgroup runs per CU.
    xcds: Accelerator complex dies; each has its own L2, and the grid hands
      each one a contiguous range of query blocks.
    lds_bytes: LDS per CU.
    peak_bf16_flops: Dense bf16 MFMA peak of the device.
    hbm_bw_bytes: HBM bandwidth, bytes/s.
  """

  name: str
  arch: str
  compute_units: int
  xcds: int
  lds_bytes: int
  peak_bf16_flops: float
  hbm_bw_bytes: float


# MI355X, used off a GPU host (the reference falls back to its V7_SPEC the
# same way, kernels/block_sizes.py:172-182, 210-240).
MI355X_SPEC = GpuSpec(name="AMD Instinct MI355X", arch="gfx950",
                      compute_units=256, xcds=8, lds_bytes=160 * 1024,
                      peak_bf16_flops=2.5e15, hbm_bw_bytes=8.0e12)


def spec_from_device(index: int = 0) -> GpuSpec:
  """The GpuSpec of torch device ``cuda:index`` (CU count and name queried;
  the rest are gfx950 constants)."""
  import torch
  props = torch.cuda.get_device_properties(index)
  arch = getattr(props, "gcnArchName", MI355X_SPEC.arch).split(":")[0]
  return dataclasses.replace(MI355X_SPEC, name=props.name, arch=arch,
                             compute_units=int(props.multi_processor_count))


def detect_spec() -> GpuSpec:
  """The GpuSpec of the current GPU, or ``MI355X_SPEC`` without one."""
  import torch
  if not torch.cuda.is_available():
    _logger.warning("No GPU detected; falling back to the %s spec.",
                    MI355X_SPEC.name)
    return MI355X_SPEC
  spec = spec_from_device(torch.cuda.current_device())
  if spec.arch != MI355X_SPEC.arch:
    _logger.warning("Device %s is %s; the kernels are built for %s.",
                    spec.name, spec.arch, MI355X_SPEC.arch)
  return spec


class BlockSizes(NamedTuple):
  block_q: int
  block_kv: int
  block_kv_compute: int


def local_blocks(q_seq_len: int, kv_seq_len: int, block_q: int,
                 block_kv: int, block_kv_compute: int) -> BlockSizes:
  """Clamps requested blocks to one call's extents, as the reference does
  before its kernel (kernels/splash.py:529-563): each block at most its
  extent, and one compute step when the clamped K/V block is not a
  multiple of the compute block."""
  for name, val in (("block_q", block_q), ("block_kv", block_kv),
                    ("block_kv_compute", block_kv_compute),
                    ("q_seq_len", q_seq_len), ("kv_seq_len", kv_seq_len)):
    if int(val) <= 0:
      raise ValueError(f"{name} must be positive, got {val}")
  bkv = min(block_kv, kv_seq_len)
  bkv_compute = min(block_kv_compute, kv_seq_len)
  if bkv % bkv_compute:
    bkv_compute = bkv
  return BlockSizes(min(block_q, q_seq_len), bkv, bkv_compute)


# The kernel's own tile, returned where the reference returns its defaults
# (kernels/block_sizes.py:534).
DEFAULT_BLOCKS = {"block_q": ROWS_PER_WORKGROUP, "block_kv": KEYS_PER_TILE,
                  "block_kv_compute": KEYS_PER_TILE}


def autotune_block_sizes(seq_len: int, head_dim: int = 128,
                         bytes_per_element: int = 2,
                         spec: GpuSpec | None = None,
                         kv_seq_len: int | None = None,
                         kernel_mode: str = "online") -> dict[str, int]:
  """The gfx950 tile for a shape (kernels/block_sizes.py:442-529): the
  fixed 256 x 64 tile, clamped to the extents.  ``spec``,
  ``bytes_per_element`` and ``kernel_mode`` do not change it (every kernel
  variant, fixed-m, residual and E4M3 keys included, runs the same tile);
  they are accepted for the reference's signature."""
  del bytes_per_element, spec, kernel_mode
  if head_dim % 8:
    raise NotImplementedError(
        f"head_dim must be a multiple of 8, got {head_dim}")
  kv = seq_len if kv_seq_len is None else kv_seq_len
  return local_blocks(seq_len, kv, **DEFAULT_BLOCKS)._asdict()


def resolve_block_sizes(seq_len: int, kv_seq_len: int, head_dim: int,
                        pinned: Mapping[str, int | None], kernel_mode: str,
                        spec: GpuSpec) -> Mapping[str, int]:
  """Blocks for one attention call: pinned, else tuned, else default, each
  field on its own (kernels/block_sizes.py:537-577)."""
  tuned = autotune_block_sizes(seq_len, head_dim=head_dim, spec=spec,
                               kv_seq_len=kv_seq_len, kernel_mode=kernel_mode)
  return {
      field: next(v for v in (pinned.get(field), tuned.get(field), default)
                  if v is not None)
      for field, default in DEFAULT_BLOCKS.items()
  }


def ring_step_blocks(shard: int, head_dim: int, *, spec: GpuSpec,
                     use_fixed_m: bool = False, qk_fp8: bool = False,
                     pinned: Mapping[str, int | None] | None = None
                     ) -> dict[str, int]:
  """Blocks for one ring step's residual call (kernels/block_sizes.py:
  587-620)."""
  mode = ("residual-qkfp8" if qk_fp8 else
          "residual-fixedm" if use_fixed_m else "residual")
  return dict(resolve_block_sizes(shard, shard, head_dim, pinned or {}, mode,
                                  spec))


def rank_block_candidates(seq_len: int, head_dim: int = 128,
                          bytes_per_element: int = 2,
                          spec: GpuSpec | None = None,
                          kv_seq_len: int | None = None,
                          top_k: int = 8) -> list[dict[str, int]]:
  """Candidate blocks ranked by cost (kernels/block_sizes.py:623-703): with
  one tile there is one candidate."""
  if top_k < 1:
    raise ValueError(f"top_k must be positive, got {top_k}")
  return [autotune_block_sizes(seq_len, head_dim, bytes_per_element, spec,
                               kv_seq_len)]


@dataclasses.dataclass(frozen=True)
class LaunchPlan:
  """What ``dt_flash_fwd_ex`` runs for a shape on the current device.

  Attributes:
    compute_units: CUs of the device (workgroups per round).
    query_blocks: 256-row query blocks, B * H * ceil(Sq / 256).
    key_tiles: 64-key tiles each block sweeps.
    rounds: query_blocks / compute_units.
    split_parts: parts each tail block runs as (1: no split).
    tail_blocks: query blocks of the last round that are split.
    whole_blocks: query blocks run over all their keys.
    workspace_bytes: workspace the plan uses.
  """

  compute_units: int
  query_blocks: int
  key_tiles: int
  rounds: float
  split_parts: int
  tail_blocks: int
  whole_blocks: int
  workspace_bytes: int


def launch_plan(batch: int, heads: int, seq_len: int,
                kv_seq_len: int | None = None, head_dim: int = 128, *,
                kv_len: int | None = None, qk_fp8: bool = False,
                workspace_bytes: int | None = None) -> LaunchPlan:
  """The launch plan of one attention call on the current GPU.

  ``workspace_bytes``: the workspace the call would pass (None: as much as
  the best plan uses, which is what ``attention`` allocates).  Head dims
  other than 64 and 128 (and every head dim with ``qk_fp8``) run
  zero-padded to the kernel's, so they plan as that dim.
  """
  from diffusers_tpu_amd import _lib
  from diffusers_tpu_amd.kernels.splash import kernel_head_dim
  if head_dim % 8:
    raise NotImplementedError(
        f"head_dim must be a multiple of 8, got {head_dim}")
  skv = seq_len if kv_seq_len is None else kv_seq_len
  d = kernel_head_dim(head_dim, qk_fp8)
  if d is None:
    raise NotImplementedError(f"head_dim {head_dim} above the kernels' "
                              "(256; 128 with qk_fp8)")
  n = 0 if kv_len is None else int(kv_len)
  lib = _lib.load()
  if workspace_bytes is None:
    workspace_bytes = lib.dt_flash_fwd_workspace_bytes(batch, heads, seq_len,
                                                       skv, n, d)
  plan = (ctypes.c_int32 * 6)()
  need = ctypes.c_size_t(0)
  _lib.check("dt_flash_fwd_plan", lib.dt_flash_fwd_plan(
      batch, heads, seq_len, skv, n, d, int(workspace_bytes), plan,
      ctypes.byref(need)))
  return LaunchPlan(compute_units=plan[0], query_blocks=plan[1],
                    key_tiles=plan[2], rounds=plan[1] / plan[0],
                    split_parts=plan[3], tail_blocks=plan[4],
                    whole_blocks=plan[5], workspace_bytes=need.value)
