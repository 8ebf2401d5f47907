"""Key lengths read from device memory (the reference's traced kv_len
scalar, kernels/splash.py:583-620, models/minimax_h3/jax_server.py:271-289)
and caller-owned attention buffers (``AttentionWorkspace``).

A graph of the whole path (prologue + attention) is captured once at the I1
shape and replayed with two lengths written into the device scalar between
replays; each replay is checked against the float64 oracle at that length.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import (assert_attn_close, assert_prologue_close, banner,
                         seeded, to64)
from oracle import attention as A
from oracle import fixed_m as FM
from oracle import norm_rope as NR

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _check_attention(out, qa, ka, v, n, rows, heads, what):
  for b in range(out.shape[0]):
    for h in heads:
      want = A.attention_f64(to64(qa[b, h, rows])[None, None],
                             to64(ka[b, h])[None, None],
                             to64(v[b, h])[None, None], kv_len=n)[0, 0]
      assert_attn_close(to64(out[b, h, rows]), want, f"{what} b{b} h{h}")


def test_graph_replays_with_two_lengths_i1(dta):
  """I1 (B2 H24 S4608 D128): prologue + attention captured once with the
  length on the device, replayed at kv_len 4396 and 4300."""
  from diffusers_tpu_amd.workloads import WORKLOADS
  w = WORKLOADS["I1"]
  banner(f"graph, device kv_len, I1 S={w.S}")
  x = w.inputs(device="cuda")
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  v = x["v"].to(torch.bfloat16).contiguous()
  n_dev = torch.full((1,), w.S, device="cuda", dtype=torch.int32)
  qa = torch.empty((w.B, w.H, w.S, w.D), device="cuda", dtype=torch.bfloat16)
  ka, out = torch.empty_like(qa), torch.empty_like(qa)
  vz = torch.empty_like(v)
  ws = dta.splash.AttentionWorkspace().reserve(qa.shape, ka.shape, n_dev)
  # v's padded rows zeroed on the device as well (the caller contract)
  ar = torch.arange(w.S, device="cuda", dtype=torch.int32).view(1, 1, w.S, 1)

  def step():
    dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps, rope=rope,
                     q_head_scale=x["hs"], valid_len=n_dev, out=(qa, ka))
    torch.mul(v, (ar < n_dev).to(torch.bfloat16), out=vz)
    dta.attention(qa, ka, vz, kv_len=n_dev, out=out, workspace=ws)

  n_dev.fill_(4396)
  step()
  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    step()
  torch.cuda.current_stream().wait_stream(side)
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    step()
  rng = np.random.default_rng(11)
  for n in (4396, 4300, 4396):
    out.zero_()
    qa.zero_()
    n_dev.fill_(n)               # eager write between replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([rng.choice(w.S, 24, replace=False),
                                     [0, n - 1, n, w.S - 1]]))
    # prologue: rows past n zeroed, the rest against the oracle
    assert torch.all(qa[:, :, n:] == 0) and torch.all(ka[:, :, n:] == 0)
    live = rows[rows < n]
    want = NR.qk_norm_rope_f64(to64(x["q"][:, live]), x["wq"].cpu().numpy(),
                               w.eps, w.positions()[live], w.axis_dims,
                               w.theta, w.mode,
                               head_scale=None if x["hs"] is None
                               else x["hs"].cpu().numpy())
    assert_prologue_close(to64(qa[:, :, live].transpose(1, 2)), want,
                          f"replay kv_len={n} prologue")
    _check_attention(out, qa, ka, vz, n, rows, (0, w.H - 1),
                     f"replay kv_len={n}")


def test_device_length_matches_host_length(dta):
  """Packed V + the tail split (S = 40000) with the length on the device
  against the same call with a host int; the packed tiles below the length
  are bit-equal."""
  sp = dta.splash
  s, n = 40000, 38990
  banner(f"device kv_len packed V S={s} n={n}")
  q = seeded((1, 2, s, 128), 301)
  k = seeded((1, 2, s, 128), 302)
  v = seeded((1, 2, s, 128), 303)
  n_dev = torch.tensor([n], device="cuda", dtype=torch.int32)
  vt_h, tiles_h = sp.pack_v(v, n)
  vt_d, tiles_d = sp.pack_v(v, n_dev)
  assert tiles_d == (s + 63) // 64 and tiles_h == (n + 63) // 64
  a = vt_h.view(2, tiles_h, -1)
  bdev = vt_d.view(2, tiles_d, -1)[:, :tiles_h]
  assert torch.equal(a, bdev)
  got = sp.attention(q, k, v, kv_len=n_dev)
  ref = sp.attention(q, k, v, kv_len=n)
  rows = np.array([0, 1, 777, 20000, s - 1])
  _check_attention(got, q, k, v, n, rows, (0, 1), "device kv_len")
  assert_attn_close(to64(got), to64(ref), "device vs host kv_len")
  # residual form
  o32, m, l = sp.residual_attention(q, k, v, kv_len=n_dev)
  o2, m2, l2 = sp.residual_attention(q, k, v, kv_len=n)
  norm = lambda o, m_, l_: to64(o) / to64(l_)
  assert_attn_close(norm(o32, m, l), norm(o2, m2, l2), "residual device len")


def test_device_length_short_and_d64(dta):
  """A device length inside the first tile, and the D = 64 kernel."""
  sp = dta.splash
  for d, s, n in ((128, 700, 5), (64, 1000, 333), (64, 1000, 1000)):
    banner(f"device kv_len d={d} s={s} n={n}")
    q = seeded((1, 3, s, d), 310 + d)
    k = seeded((1, 3, s, d), 311 + d)
    v = seeded((1, 3, s, d), 312 + d)
    n_dev = torch.tensor([n], device="cuda", dtype=torch.int64)
    got = sp.attention(q, k, v, kv_len=n_dev)
    want = A.attention_f64(to64(q), to64(k), to64(v), kv_len=n)
    assert_attn_close(to64(got), want, f"d{d} n{n}")


def test_device_length_smoothing_and_fixed_m(dta):
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  from diffusers_tpu_amd.kernels import k_smoothing
  b, h, s, d, n = 1, 4, 3000, 128, 2711
  banner(f"device kv_len smoothing s={s} n={n}")
  q = seeded((b, h, s, d), 320)
  k = seeded((b, h, s, d), 321)
  n_dev = torch.tensor([n], device="cuda", dtype=torch.int32)
  ks = k_smoothing.smooth_keys(k, n_dev)
  want, mean = FM.smooth_keys(to64(k), n)
  diff = np.abs(to64(ks) - want)
  # float32 means summed in another chunk order than the oracle's float64
  # one: a result may move by one bf16 step of the mean near a boundary
  assert (diff <= 2.0 ** -8 * (np.abs(mean) + np.abs(want)) + 1e-30).all()
  ks2, mk = fmb.fixed_m_prepare(q, k, kv_len=n_dev, smooth=True)
  ks3, mk3 = fmb.fixed_m_prepare(q, k, kv_len=n, smooth=True)
  assert torch.equal(mk[1], mk3[1])
  assert (mk[0] - mk3[0]).abs().max().item() <= 1.0
  assert torch.all(ks2[:, :, n:] == 0)
  assert_attn_close(to64(ks2), to64(ks3), "smoothed keys device vs host")


def test_workspace_reuse_is_bit_equal(dta):
  """Two calls through one AttentionWorkspace (packed V + split, then a
  smaller shape) equal fresh-allocation calls bit for bit."""
  sp = dta.splash
  ws = sp.AttentionWorkspace()
  banner("AttentionWorkspace reuse")
  for s, n, hq in ((40000, 39000, 2), (36000, None, 1), (5000, 4321, 3)):
    q = seeded((1, hq, s, 128), 330 + s % 97)
    k = seeded((1, hq, s, 128), 331 + s % 97)
    v = seeded((1, hq, s, 128), 332 + s % 97)
    fresh = sp.attention(q, k, v, kv_len=n)
    out = torch.empty_like(q)
    r1 = sp.attention(q, k, v, kv_len=n, out=out, workspace=ws)
    assert r1 is out and torch.equal(out, fresh)
    r2 = sp.attention(q, k, v, kv_len=n, workspace=ws)
    assert torch.equal(r2, fresh)
    o32, m, l = sp.residual_attention(q, k, v, kv_len=n, workspace=ws)
    f32, fm, fl = sp.residual_attention(q, k, v, kv_len=n)
    assert torch.equal(o32, f32) and torch.equal(m, fm) and torch.equal(l, fl)
  assert ws._vt is not None and ws._split is not None


def test_workspace_must_match_the_tensors(dta):
  """A workspace of another device or type is refused before any launch."""
  sp = dta.splash
  banner("AttentionWorkspace device check")
  q = seeded((1, 1, 300, 128), 340)
  with pytest.raises(ValueError):
    sp.attention(q, q, q, workspace=sp.AttentionWorkspace(device="cpu"))
  with pytest.raises(TypeError):
    sp.attention(q, q, q, workspace=object())
