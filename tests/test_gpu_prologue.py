"""Parity of the gfx950 QK-RMSNorm + RoPE kernel (dt_qk_norm_rope) against
the float64 oracle (oracle/norm_rope.py) on the same bf16 inputs.

Tolerance: 1e-2 max-abs (north star) plus the final bf16 rounding of the
output, which the reference performs too (at most 2^-8 relative).
"""
import numpy as np
import pytest
import torch

from gpu_helpers import PROLOGUE_MAX_ABS, banner, seeded, to64
from oracle import norm_rope as NR

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _check(got, want, what):
  err = np.abs(got - want)
  lim = PROLOGUE_MAX_ABS + 2.0 ** -8 * np.abs(want)
  bad = err > lim
  assert not bad.any(), f"{what}: {bad.sum()} over tolerance, max {err.max():.3g}"
  return float(err.max())


def _run_case(dta, b, s, h, d, mode, dims, *, theta=1e4, eps=1e-6,
              head_scale=False, valid_len=None, layout="bhsd", seed=0):
  q = seeded((b, s, h, d), seed)
  k = seeded((b, s, h, d), seed + 1)
  g = torch.Generator().manual_seed(seed + 2)
  wq = 1 + 0.02 * torch.randn(d, generator=g)
  wk = 1 + 0.02 * torch.randn(d, generator=g)
  pos = torch.randint(-3, 100, (s, 3), generator=g, dtype=torch.int32)
  hs = (0.5 + torch.rand(h, generator=g)) if head_scale else None
  rope = None if mode == "none" else dta.RopeSpec(mode, pos.cuda(), dims, theta)
  qo, ko = dta.qk_norm_rope(q, k, wq, wk, eps=eps, rope=rope,
                            q_head_scale=None if hs is None else hs.cuda(),
                            valid_len=valid_len, out_layout=layout)
  torch.cuda.synchronize()
  if layout == "bhsd":
    qo, ko = qo.transpose(1, 2), ko.transpose(1, 2)
  wantq = NR.qk_norm_rope_f64(to64(q), wq.numpy(), eps, pos.numpy(), dims,
                              theta, mode, head_scale=None if hs is None
                              else hs.numpy(), valid_len=valid_len)
  wantk = NR.qk_norm_rope_f64(to64(k), wk.numpy(), eps, pos.numpy(), dims,
                              theta, mode, valid_len=valid_len)
  _check(to64(qo), wantq, "q")
  _check(to64(ko), wantk, "k")
  if valid_len is not None:
    assert torch.all(qo[:, valid_len:] == 0) and torch.all(ko[:, valid_len:] == 0)


CASES = [
    # (b, s, h, d, mode, axis_dims, kwargs)
    (1, 1024, 8, 64, "half", (64, 0, 0), {}),                 # plumbing: 1D
    (2, 300, 24, 128, "half", (0, 64, 64), {}),               # image: 2D
    (1, 257, 40, 128, "half", (44, 42, 42), {}),              # video: 3D
    (1, 200, 5, 128, "half", (44, 42, 42), {"head_scale": True}),  # V7 shard
    (1, 130, 6, 128, "half", (32, 32, 32), {"eps": 1e-5}),    # H3 96-lane rope
    (1, 99, 7, 128, "pair", (16, 56, 56), {}),                # Qwen pairs
    (1, 64, 3, 64, "pair", (20, 22, 22), {}),
    (2, 77, 4, 128, "none", (0, 0, 0), {}),                   # norm only
    (1, 300, 4, 128, "half", (0, 64, 64), {"valid_len": 211}),  # padding
    (1, 100, 3, 128, "half", (44, 42, 42), {"layout": "bshd"}),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[4]}-{c[5]}-{c[1]}x{c[2]}x{c[3]}"
                                             f"-{sorted(c[6])}" for c in CASES])
def test_prologue_matches_oracle(dta, case):
  b, s, h, d, mode, dims, kw = case
  banner(f"prologue {case}")
  _run_case(dta, b, s, h, d, mode, dims, **kw)


def test_prologue_strided_input_and_inplace(dta):
  """q and k as views of one fused qkv projection (B, S, 3, H, D)."""
  banner("prologue strided / in-place")
  b, s, h, d = 1, 150, 4, 128
  qkv = seeded((b, s, 3, h, d), 7)
  q, k = qkv[:, :, 0], qkv[:, :, 1]
  wq, wk = torch.ones(d), torch.ones(d)
  pos = torch.zeros((s, 3), dtype=torch.int32)
  pos[:, 0] = torch.arange(s)
  rope = dta.RopeSpec("half", pos.cuda(), (128, 0, 0), 1e4)
  a = dta.qk_norm_rope(q, k, wq, wk, rope=rope, out_layout="bshd")
  qc, kc = q.contiguous(), k.contiguous()
  bq, bk = dta.qk_norm_rope(qc, kc, wq, wk, rope=rope, out_layout="bshd")
  torch.cuda.synchronize()
  assert torch.equal(a[0], bq) and torch.equal(a[1], bk)
  # in place on contiguous tensors
  dta.qk_norm_rope(qc, kc, wq, wk, rope=rope, out_layout="bshd",
                   out=(qc, kc))
  torch.cuda.synchronize()
  assert torch.equal(qc, bq) and torch.equal(kc, bk)


def test_prologue_identity_rows(dta):
  """Position (0,0,0) rows are RMSNorm only (text rows, jax_dit.py:727-731)."""
  banner("prologue identity rows")
  b, s, h, d = 1, 64, 2, 128
  q = seeded((b, s, h, d), 3)
  w = torch.ones(d)
  pos = torch.zeros((s, 3), dtype=torch.int32)
  rope = dta.RopeSpec("half", pos.cuda(), (44, 42, 42), 1e4)
  a = dta.qk_norm_rope(q, q, w, w, rope=rope)
  b_ = dta.qk_norm_rope(q, q, w, w, rope=None)
  torch.cuda.synchronize()
  assert torch.equal(a[0], b_[0])
