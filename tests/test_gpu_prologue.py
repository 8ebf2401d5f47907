"""Parity of the gfx950 QK-RMSNorm + RoPE kernel (dt_qk_norm_rope) against
the float64 oracle (oracle/norm_rope.py) on the same bf16 inputs.

Tolerance: the kernel's arithmetic error, with the final bf16 rounding of
the output taken out (how far the float64 oracle value lies outside the
rounding interval of the bf16 result), within the north-star 1e-2 max-abs.
(A flat 1e-2 against bf16(oracle)
cannot hold for any bf16 implementation: where the exact value sits on a
rounding boundary, float32 rounding noise picks the neighbour, one bf16
step = 0.0156 at |x| in [2, 4).)
"""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_prologue_close, banner, seeded, to64
from oracle import norm_rope as NR

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _check(got, want, what):
  return assert_prologue_close(got, want, what)["kernel"]


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


# ------------------------------------------------------ table-driven rotation


@pytest.mark.parametrize("mode,dims", [("half", (44, 42, 42)),
                                       ("half", (32, 32, 32)),
                                       ("pair", (16, 56, 56)),
                                       ("pair", (20, 22, 22))])
def test_table_equals_positions(dta, mode, dims):
  """cos/sin of the positional angles as a table reproduce the positions
  path to within the sin/cos approximation (both round to bf16 at the end)."""
  banner(f"prologue table vs positions {mode} {dims}")
  d = 128 if sum(dims) > 64 else 64
  b, s, h = 2, 190, 5
  q, k = seeded((b, s, h, d), 20), seeded((b, s, h, d), 21)
  w = 1 + 0.02 * torch.randn(d, generator=torch.Generator().manual_seed(22))
  pos = torch.randint(-3, 200, (s, 3), dtype=torch.int32,
                      generator=torch.Generator().manual_seed(23))
  ang = torch.from_numpy(NR.rope_angles_f64(pos.numpy(), dims, 1e4))
  tab = dta.RopeTable(mode, torch.cos(ang).float().cuda(),
                      torch.sin(ang).float().cuda())
  a = dta.qk_norm_rope(q, k, w, w, rope=tab)
  p_ = dta.qk_norm_rope(q, k, w, w,
                        rope=dta.RopeSpec(mode, pos.cuda(), dims, 1e4))
  torch.cuda.synchronize()
  for x, y in zip(a, p_):
    err = (x.float() - y.float()).abs()
    assert (err <= 2e-3 + 2.0 ** -7 * y.float().abs()).all(), err.max()
  want = NR.qk_norm_rope_table_f64(to64(q), w.numpy(), 1e-6, np.cos(ang.numpy()),
                                   np.sin(ang.numpy()), mode)
  _check(to64(a[0].transpose(1, 2)), want, "q table")


def test_table_h3_cos_sin(dta):
  """H3's apply_rope operands: (S, 96) cos/sin with repeated halves,
  eps 1e-5, head dim 128 (models/minimax_h3/jax_dit.py:251-262)."""
  banner("prologue table H3 cos/sin")
  from diffusers_tpu_amd.kernels.qk_norm_rope import check_halves
  b, s, h, d = 1, 300, 6, 128
  q, k = seeded((b, s, h, d), 30), seeded((b, s, h, d), 31)
  g = torch.Generator().manual_seed(32)
  wq, wk = 1 + 0.02 * torch.randn(d, generator=g), torch.ones(d)
  ang = torch.rand(s, 48, generator=g, dtype=torch.float64) * 50
  cos = torch.cos(torch.cat([ang, ang], -1)).float()
  sin = torch.sin(torch.cat([ang, ang], -1)).float()
  assert check_halves(cos, sin)
  tab = dta.RopeTable.from_cos_sin(cos.cuda(), sin.cuda())
  qo, ko = dta.qk_norm_rope(q, k, wq, wk, eps=1e-5, rope=tab, valid_len=250)
  torch.cuda.synchronize()
  for x, w, got in ((q, wq, qo), (k, wk, ko)):
    want = NR.h3_apply_rope_f64(NR.rms_norm_f64(to64(x), w.numpy(), 1e-5),
                                cos.double().numpy(), sin.double().numpy())
    want[:, 250:] = 0
    _check(to64(got.transpose(1, 2)), want, "H3 table")


def test_table_moss_rows_per_batch(dta):
  """MOSS's (B, S, D) [sin | cos] operand, different per batch item and in
  bf16 as the model passes it (models/moss_image/jax_dit.py:136-142,233)."""
  banner("prologue table MOSS rows")
  b, s, h, d = 2, 257, 4, 128
  q, k = seeded((b, s, h, d), 40), seeded((b, s, h, d), 41)
  g = torch.Generator().manual_seed(42)
  ang = torch.rand(b, s, 64, generator=g, dtype=torch.float64) * 30
  rows = torch.cat([torch.sin(ang), torch.cos(ang)], -1).to(torch.bfloat16)
  w = 1 + 0.02 * torch.randn(d, generator=g)
  hs = 0.5 + torch.rand(h, generator=g)
  tab = dta.RopeTable.from_sin_cos_rows(rows.cuda())
  qo, ko = dta.qk_norm_rope(q, k, w, w, rope=tab, q_head_scale=hs.cuda(),
                            out_layout="bshd")
  torch.cuda.synchronize()
  r64 = to64(rows)
  wantq = NR.moss_rotate_f64(NR.rms_norm_f64(to64(q), w.numpy(), 1e-6), r64)
  wantq = wantq * hs.double().numpy()[None, None, :, None]
  wantk = NR.moss_rotate_f64(NR.rms_norm_f64(to64(k), w.numpy(), 1e-6), r64)
  _check(to64(qo), wantq, "MOSS q")
  _check(to64(ko), wantk, "MOSS k")


def test_table_partial_rotary_and_d64(dta):
  """Rotary narrower than the head (rotate-half 32 of 64 channels, pairs 40
  of 64): channels past it pass through; a (1, S, n) table broadcasts."""
  banner("prologue table partial rotary D=64")
  b, s, h, d = 2, 100, 3, 64
  q = seeded((b, s, h, d), 50)
  w = torch.ones(d)
  g = torch.Generator().manual_seed(51)
  # (mode, pairs, table row width): pairs 18 splits a lane chunk (per-element
  # reads); width 18 > 16 makes rows 8-byte aligned only (per-element reads)
  for mode, half, width in (("half", 16, 16), ("pair", 20, 20),
                            ("pair", 18, 18), ("half", 16, 18)):
    ang = torch.rand(1, s, width, generator=g, dtype=torch.float64) * 9
    tab = dta.RopeTable(mode, torch.cos(ang).float().cuda()[..., :half],
                        torch.sin(ang).float().cuda()[..., :half])
    ang = ang[..., :half]
    qo, _ = dta.qk_norm_rope(q, q, w, w, rope=tab, out_layout="bshd")
    torch.cuda.synchronize()
    want = NR.qk_norm_rope_table_f64(to64(q), w.numpy(), 1e-6,
                                     np.cos(ang[0].numpy()),
                                     np.sin(ang[0].numpy()), mode)
    _check(to64(qo), want, f"partial {mode}")


def test_table_rejects_bad_operands(dta):
  banner("prologue table errors")
  q = seeded((1, 16, 2, 128), 60)
  w = torch.ones(128)
  c = torch.ones(16, 12, device="cuda")
  with pytest.raises(Exception, match="rotate-half"):
    dta.qk_norm_rope(q, q, w, w, rope=dta.RopeTable("half", c, c))
  with pytest.raises(ValueError):
    dta.qk_norm_rope(q, q, w, w,
                     rope=dta.RopeTable("half", torch.ones(15, 16,
                                                           device="cuda"),
                                        torch.ones(15, 16, device="cuda")))
  with pytest.raises(Exception):
    big = torch.ones(16, 72, device="cuda")
    dta.qk_norm_rope(q, q, w, w, rope=dta.RopeTable("pair", big, big))


F32_CASES = [
    # (b, s, h, d, mode, axis_dims, kwargs)
    (1, 1024, 8, 64, "half", (64, 0, 0), {}),                 # plumbing config
    (1, 257, 5, 128, "half", (44, 42, 42), {"head_scale": True}),
    (1, 99, 7, 128, "pair", (16, 56, 56), {"valid_len": 60}),
    (2, 77, 4, 128, "none", (0, 0, 0), {}),
]


@pytest.mark.parametrize("case", F32_CASES,
                         ids=[f"f32-{c[4]}-{c[1]}x{c[2]}x{c[3]}" for c in F32_CASES])
def test_prologue_fp32_inputs(dta, case):
  """fp32 q and k go through dt_qk_norm_rope_f32, which reads them as fp32:
  the output is the correctly rounded oracle of the fp32 values almost
  everywhere (a bf16 cast of the inputs first would miss it on a large
  share of the elements)."""
  b, s, h, d, mode, dims, kw = case
  banner(f"prologue fp32 inputs {case}")
  g = torch.Generator().manual_seed(40)
  q = torch.randn((b, s, h, d), generator=g).cuda()
  k = torch.randn((b, s, h, d), generator=g).cuda()
  wq = 1 + 0.02 * torch.randn(d, generator=g)
  wk = 1 + 0.02 * torch.randn(d, generator=g)
  pos = torch.randint(-3, 100, (s, 3), generator=g, dtype=torch.int32)
  hs = (0.5 + torch.rand(h, generator=g)) if kw.get("head_scale") else None
  vl = kw.get("valid_len")
  rope = None if mode == "none" else dta.RopeSpec(mode, pos.cuda(), dims, 1e4)
  qo, ko = dta.qk_norm_rope(q, k, wq, wk, rope=rope, valid_len=vl,
                            q_head_scale=None if hs is None else hs.cuda())
  torch.cuda.synchronize()
  qo, ko = qo.transpose(1, 2), ko.transpose(1, 2)
  wantq = NR.qk_norm_rope_f64(to64(q), wq.numpy(), 1e-6, pos.numpy(), dims,
                              1e4, mode, valid_len=vl,
                              head_scale=None if hs is None else hs.numpy())
  wantk = NR.qk_norm_rope_f64(to64(k), wk.numpy(), 1e-6, pos.numpy(), dims,
                              1e4, mode, valid_len=vl)
  for got, want, nm in ((qo, wantq, "q"), (ko, wantk, "k")):
    e = assert_prologue_close(to64(got), want, f"fp32 {nm}")
    assert e["exact"] >= 0.99, f"fp32 {nm}: {e['exact']:.4f} correctly rounded"
  # the bf16 entry on the same values rounds the inputs first
  qb, _ = dta.qk_norm_rope(q.to(torch.bfloat16), k.to(torch.bfloat16), wq, wk,
                           rope=rope, valid_len=vl,
                           q_head_scale=None if hs is None else hs.cuda())
  torch.cuda.synchronize()
  from gpu_helpers import prologue_errors
  assert prologue_errors(to64(qb.transpose(1, 2)), wantq)["exact"] < 0.9


@pytest.mark.parametrize("mode,dims,d", [("half", (44, 42, 42), 128),
                                         ("pair", (16, 56, 56), 128),
                                         ("half", (64, 0, 0), 64)])
def test_table_fp32_inputs(dta, mode, dims, d):
  """fp32 q and k with a cos/sin table go through
  dt_qk_norm_rope_table_f32: against the table oracle of the fp32 values,
  within 1e-2 and correctly rounded almost everywhere, and equal to the
  positions path on the same fp32 inputs to within the sin/cos
  approximation."""
  banner(f"prologue table fp32 inputs {mode} {dims}")
  b, s, h = 2, 211, 5
  g = torch.Generator().manual_seed(50)
  q = torch.randn((b, s, h, d), generator=g).cuda()
  k = torch.randn((b, s, h, d), generator=g).cuda()
  w = 1 + 0.02 * torch.randn(d, generator=g)
  pos = torch.randint(-3, 200, (s, 3), dtype=torch.int32, generator=g)
  ang = NR.rope_angles_f64(pos.numpy(), dims, 1e4)
  tab = dta.RopeTable(mode, torch.from_numpy(np.cos(ang)).float().cuda(),
                      torch.from_numpy(np.sin(ang)).float().cuda())
  qo, ko = dta.qk_norm_rope(q, k, w, w, rope=tab, valid_len=200)
  pq, pk = dta.qk_norm_rope(q, k, w, w, valid_len=200,
                            rope=dta.RopeSpec(mode, pos.cuda(), dims, 1e4))
  torch.cuda.synchronize()
  for x, got, ref in ((q, qo, pq), (k, ko, pk)):
    want = NR.qk_norm_rope_table_f64(to64(x), w.numpy(), 1e-6, np.cos(ang),
                                     np.sin(ang), mode)
    want[:, 200:] = 0
    e = assert_prologue_close(to64(got.transpose(1, 2)), want, "fp32 table")
    assert e["exact"] >= 0.99, f"{e['exact']:.4f} correctly rounded"
    err = (got.float() - ref.float()).abs()
    assert (err <= 2e-3 + 2.0 ** -7 * ref.float().abs()).all(), err.max()
