"""Per-sample key lengths in one call, and the range of device lengths.

The reference's MOSS CFG path takes ``kv_len`` as a ``[B]`` vector: it masks
``arange(S) < kv_len[:, None]``, smooths each sample's keys over its own real
rows and loops B single-sample kernel calls
(models/moss_image/jax_dit.py:181-210, mask :185, smoothing :195-196, loop
:198-202).  Here the lengths are one device ``int32[B]`` (or a host list)
that every kernel indexes by batch element, so a CFG pair whose prompts
differ in length is one launch per stage.  Each sample is checked against
the float64 oracle at its own length.

A device length <= 0 gives the empty result (zero rows; residual
o = m = l = 0) and one above the sequence is clamped to it.
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


def _count_calls(monkeypatch, name):
  """Counts the C-ABI calls of ``name`` made through the ctypes binding."""
  from diffusers_tpu_amd import _lib
  lib = _lib.load()
  fn = getattr(lib, name)
  calls = []

  def wrapped(*args):
    calls.append(1)
    return fn(*args)
  monkeypatch.setattr(lib, name, wrapped)
  return calls


def _smooth_ok(got, k64, n):
  """Smoothed keys of one sample against the float64 oracle at length n
  (float32 means summed in another order than the oracle's float64 one: a
  value may move by one bf16 step of the mean near a rounding boundary)."""
  want, mean = FM.smooth_keys(k64, n)
  diff = np.abs(got - want)
  assert (diff <= 2.0 ** -8 * (np.abs(mean) + np.abs(want)) + 1e-30).all()


def test_i1_cfg_pair_per_sample_lengths(dta, monkeypatch):
  """I1 (B2 H24 S4608 D128) with the two samples at 4396 and 4233 real
  tokens: prologue zeroing, per-sample key smoothing and attention, each one
  launch over both samples, against the oracle per sample."""
  from diffusers_tpu_amd.kernels import k_smoothing
  from diffusers_tpu_amd.workloads import WORKLOADS
  w = WORKLOADS["I1"]
  lens = (4396, 4233)
  banner(f"per-sample lengths I1 {lens}")
  x = w.inputs(device="cuda")
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  n_dev = torch.tensor(lens, device="cuda", dtype=torch.int32)
  qa, ka = dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps,
                            rope=rope, valid_len=n_dev)
  qh, kh = dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps,
                            rope=rope, valid_len=list(lens))
  assert torch.equal(qa, qh) and torch.equal(ka, kh)
  # prologue: sampled tokens around both lengths, every head, per sample
  rows = np.array([0, 1, 2047, 4095, 4096, 4232, 4233, 4300, 4395, 4396,
                   4607])
  pos = x["pos"].cpu().numpy()
  for b, n in enumerate(lens):
    for name, src, wt in (("q", x["q"], x["wq"]), ("k", x["k"], x["wk"])):
      want = NR.qk_norm_rope_f64(to64(src[b:b + 1, rows]), to64(wt), w.eps,
                                 pos[rows], w.axis_dims, w.theta, w.mode)
      want[:, rows >= n] = 0.0
      got = to64((qa if name == "q" else ka)[b, :, rows]).transpose(1, 0, 2)
      assert_prologue_close(got[None], want, f"prologue {name} b{b}")
      assert not got[rows >= n].any()
  # v zeroed per sample, as the caller contract asks
  v = x["v"].clone()
  for b, n in enumerate(lens):
    v[b, :, n:] = 0
  # key smoothing: each sample's mean over its own real rows
  ks = k_smoothing.smooth_keys(ka, n_dev)
  assert torch.equal(ks, k_smoothing.smooth_keys(ka, list(lens)))
  for b, n in enumerate(lens):
    for h in (0, 13, 23):
      _smooth_ok(to64(ks[b:b + 1, h:h + 1]), to64(ka[b:b + 1, h:h + 1]), n)
  # attention: one launch for the pair
  calls = _count_calls(monkeypatch, "dt_flash_fwd_ex")
  out = dta.attention(qa, ks, v, kv_len=n_dev)
  assert len(calls) == 1
  out_h = dta.attention(qa, ks, v, kv_len=list(lens))
  assert len(calls) == 2
  assert torch.equal(out, out_h)
  for b, n in enumerate(lens):
    for h in (0, 7, 23):
      want = A.attention_f64(to64(qa[b, h, rows])[None, None],
                             to64(ks[b, h])[None, None],
                             to64(v[b, h])[None, None], kv_len=n)[0, 0]
      assert_attn_close(to64(out[b, h, rows]), want, f"attention b{b} h{h}")


def test_per_sample_packed_v_split_gqa(dta):
  """Packed V (S = 40000) with the tail split, GQA 4:2, residual outputs,
  lengths 39000 and 33333, against the oracle per sample and against
  single-sample calls at the same length."""
  sp = dta.splash
  s, lens = 40000, (39000, 33333)
  banner(f"per-sample lengths packed V S={s} {lens}")
  q = seeded((2, 4, s, 128), 401)
  k = seeded((2, 2, s, 128), 402)
  v = seeded((2, 2, s, 128), 403)
  for b, n in enumerate(lens):
    k[b, :, n:] = 0
    v[b, :, n:] = 0
  n_dev = torch.tensor(lens, device="cuda", dtype=torch.int32)
  out = sp.attention(q, k, v, kv_len=n_dev)
  o32, m, l = sp.residual_attention(q, k, v, kv_len=n_dev)
  rows = np.array([0, 5, 12345, 30000, s - 1])
  for b, n in enumerate(lens):
    one = sp.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], kv_len=n)
    assert_attn_close(to64(out[b]), to64(one[0]), f"vs single call b{b}")
    for h in (0, 3):
      want = A.attention_f64(to64(q[b, h, rows])[None, None],
                             to64(k[b, h // 2])[None, None],
                             to64(v[b, h // 2])[None, None], kv_len=n)[0, 0]
      assert_attn_close(to64(out[b, h, rows]), want, f"packed b{b} h{h}")
      norm = to64(o32[b, h, rows]) / to64(l[b, h, rows])
      assert_attn_close(norm, want, f"residual b{b} h{h}")


def test_per_sample_d64_and_fixed_m(dta):
  """The D = 64 kernel and the fixed-m preparation with per-sample
  lengths."""
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  sp = dta.splash
  s, lens = 3000, (2999, 1000, 17)
  banner(f"per-sample lengths D=64 {lens}")
  q = seeded((3, 2, s, 64), 411)
  k = seeded((3, 2, s, 64), 412)
  v = seeded((3, 2, s, 64), 413)
  n_dev = torch.tensor(lens, device="cuda", dtype=torch.int64)
  out = sp.attention(q, k, v, kv_len=n_dev)
  for b, n in enumerate(lens):
    want = A.attention_f64(to64(q[b:b + 1]), to64(k[b:b + 1]),
                           to64(v[b:b + 1]), kv_len=n)
    assert_attn_close(to64(out[b:b + 1]), want, f"d64 b{b} n{n}")
  banner("per-sample lengths fixed-m prepare")
  q = seeded((2, 4, s, 128), 421)
  k = seeded((2, 4, s, 128), 422)
  lens = (2500, 2999)
  n_dev = torch.tensor(lens, device="cuda", dtype=torch.int32)
  ks, mk = fmb.fixed_m_prepare(q, k, kv_len=n_dev, smooth=True)
  for b, n in enumerate(lens):
    _smooth_ok(to64(ks[b:b + 1]), to64(k[b:b + 1]), n)
    assert not ks[b, :, n:].any()
  # the operand over both samples' smoothed keys (the largest norms of the
  # batch), compared with the host composition of the same smoothed keys
  qs = to64(q) * (1.0 / np.sqrt(128)) * FM.LOG2_E
  want = FM.fixed_m_operands(qs, to64(ks))
  got = mk.cpu().numpy()
  assert np.array_equal(got[1], want[1])
  assert np.abs(got[0] - want[0]).max() <= 1.0
  out = sp.attention(q, ks, seeded((2, 4, s, 128), 423), kv_len=n_dev,
                     use_fixed_m=True)
  assert torch.isfinite(out.float()).all()


def test_device_length_zero_and_past_the_end(dta):
  """A device length of 0 gives the empty result and one of Skv + 5 the
  full one, through attention (normalized and residual, row-major and
  packed V), the V pack, key smoothing, the fixed-m operand and the
  prologue."""
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  from diffusers_tpu_amd.kernels import k_smoothing
  sp = dta.splash
  for s, d in ((777, 128), (900, 64), (33000, 128)):
    banner(f"device length 0 / Skv+5 S={s} D={d}")
    q = seeded((2, 2, s, d), 431)
    k = seeded((2, 2, s, d), 432)
    v = seeded((2, 2, s, d), 433)
    zero = torch.tensor([0], device="cuda", dtype=torch.int32)
    past = torch.tensor([s + 5], device="cuda", dtype=torch.int32)
    mixed = torch.tensor([0, s - 100], device="cuda", dtype=torch.int32)
    assert not sp.attention(q, k, v, kv_len=zero).any()
    o32, m, l = sp.residual_attention(q, k, v, kv_len=zero)
    assert not o32.any() and not m.any() and not l.any()
    full = sp.attention(q, k, v)
    assert torch.equal(sp.attention(q, k, v, kv_len=past), full)
    out = sp.attention(q, k, v, kv_len=mixed)
    assert not out[0].any()
    want = A.attention_f64(to64(q[1:, :, :300]), to64(k[1:]), to64(v[1:]),
                           kv_len=s - 100)
    assert_attn_close(to64(out[1:, :, :300]), want, f"mixed S={s}")
    if d == 128:
      ks = k_smoothing.smooth_keys(k, zero)
      assert not ks.any()
      assert torch.equal(k_smoothing.smooth_keys(k, past),
                         k_smoothing.smooth_keys(k))
      ks, mk = fmb.fixed_m_prepare(q, k, kv_len=zero, smooth=True)
      assert not ks.any()
      assert mk[0].abs().max().item() == 0 and bool((mk[1] == 1).all())
  banner("prologue device valid_len 0 / S+5")
  b, s, h, d = 2, 300, 3, 128
  x = seeded((b, s, h, d), 441)
  y = seeded((b, s, h, d), 442)
  wt = torch.ones(d, device="cuda")
  qz, kz = dta.qk_norm_rope(x, y, wt, wt, valid_len=torch.tensor(
      [0, 200], device="cuda", dtype=torch.int32))
  assert not qz[0].any() and not kz[0].any()
  assert not qz[1, :, 200:].any() and not kz[1, :, 200:].any()
  qf, kf = dta.qk_norm_rope(x, y, wt, wt)
  assert torch.equal(qz[1, :, :200], qf[1, :, :200])
  qp, kp = dta.qk_norm_rope(x, y, wt, wt, valid_len=torch.tensor(
      [s + 5], device="cuda", dtype=torch.int32))
  assert torch.equal(qp, qf) and torch.equal(kp, kf)


def test_per_sample_lengths_in_a_replayed_graph(dta):
  """Prologue + attention captured once with a two-entry device length and
  replayed with other per-sample lengths written between replays (one of
  them 0: that sample's rows come out zero), each replay against the
  oracle per sample."""
  b, h, s, d = 2, 3, 5000, 128
  banner(f"per-sample lengths graph replay B{b} H{h} S{s}")
  x = seeded((b, s, h, d), 451)
  y = seeded((b, s, h, d), 452)
  v = seeded((b, h, s, d), 453)
  wt = 1.0 + 0.02 * seeded((d,), 454, dtype=torch.float32)
  lens = torch.tensor([s, s], device="cuda", dtype=torch.int32)
  qa = torch.empty((b, h, s, d), device="cuda", dtype=torch.bfloat16)
  ka, out, vz = torch.empty_like(qa), torch.empty_like(qa), torch.empty_like(v)
  ws = dta.splash.AttentionWorkspace().reserve(qa.shape, ka.shape, lens)
  ar = torch.arange(s, device="cuda", dtype=torch.int32).view(1, 1, s, 1)

  def step():
    dta.qk_norm_rope(x, y, wt, wt, eps=1e-6, valid_len=lens, out=(qa, ka))
    torch.mul(v, (ar < lens.view(b, 1, 1, 1)).to(torch.bfloat16), out=vz)
    dta.attention(qa, ka, vz, kv_len=lens, out=out, workspace=ws)

  step()
  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    step()
  torch.cuda.current_stream().wait_stream(side)
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    step()
  rows = np.array([0, 1, 999, 2499, 2500, 2999, 3000, 4989, 4990, s - 1])
  for pair in ((4990, 3000), (1000, s), (0, 2500)):
    out.fill_(7.0)
    lens.copy_(torch.tensor(pair, dtype=torch.int32))  # eager write
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    for bi, n in enumerate(pair):
      if n == 0:
        assert not out[bi].any() and not qa[bi].any()
        continue
      assert not qa[bi, :, n:].any() and not ka[bi, :, n:].any()
      for hh in (0, h - 1):
        want = A.attention_f64(to64(qa[bi, hh, rows])[None, None],
                               to64(ka[bi, hh])[None, None],
                               to64(vz[bi, hh])[None, None], kv_len=n)[0, 0]
        assert_attn_close(to64(out[bi, hh, rows]), want,
                          f"replay {pair} b{bi} h{hh}")


def test_per_sample_lengths_qk_fp8(dta):
  """E4M3 keys with per-sample lengths (a host list): each sample against
  the float64 softmax of its E4M3-rounded operands at its own length."""
  from oracle import fp8 as P8
  b, h, s, lens = 2, 3, 3000, [2111, 3000]
  banner(f"per-sample lengths qk_fp8 {lens}")
  q = seeded((b, h, s, 128), 461)
  k = seeded((b, h, s, 128), 462)
  v = seeded((b, h, s, 128), 463)
  got = dta.attention(q, k, v, qk_fp8=True, kv_len=lens)
  c = (1.0 / np.sqrt(128)) * np.log2(np.e)
  q8 = P8.e4m3_round(to64((q.float() * c).to(torch.bfloat16)))
  k8 = P8.e4m3_round(to64(k))
  for bi, n in enumerate(lens):
    want = A.attention_f64(q8[bi:bi + 1], k8[bi:bi + 1], to64(v[bi:bi + 1]),
                           scale=np.log(2.0), kv_len=n)
    assert_attn_close(to64(got[bi:bi + 1]), want, f"qk_fp8 b{bi} n{n}")


def test_per_sample_lengths_noalloc_entry(dta):
  """dt_flash_fwd_ex_noalloc with a two-entry device length equals
  dt_flash_fwd_ex with a caller workspace, bit for bit (packed V + split)."""
  from diffusers_tpu_amd import _lib
  sp = dta.splash
  lib = _lib.load()
  b, h, s, lens = 2, 2, 40000, (39000, 35555)
  banner(f"per-sample lengths noalloc S={s} {lens}")
  q = seeded((b, h, s, 128), 471)
  k = seeded((b, h, s, 128), 472)
  v = seeded((b, h, s, 128), 473)
  n_dev = torch.tensor(lens, device="cuda", dtype=torch.int32)
  vt, tiles = sp.pack_v(v, n_dev)
  need = lib.dt_flash_fwd_workspace_bytes(b, h, s, s, 0, 128)
  nbytes = min(need, _lib.NOALLOC_SCRATCH_BYTES)
  assert nbytes > 0
  ws = torch.empty((nbytes + 3) // 4, device="cuda", dtype=torch.float32)
  s3 = lambda t: _lib.i64_array(*t.stride()[:3])
  st = torch.cuda.current_stream().cuda_stream
  outs = []
  for fn in ("ex", "noalloc"):
    o = torch.full_like(q, float("nan"))
    common = (q.data_ptr(), k.data_ptr(), 0, None, None, vt.data_ptr(), tiles,
              o.data_ptr(), b, h, h, s, s, 128, s3(q), s3(k), s3(o),
              1.0 / 128 ** 0.5, b, n_dev.data_ptr(), None, None, None, None,
              None, None)
    if fn == "ex":
      rc = lib.dt_flash_fwd_ex(*common, ws.data_ptr(), nbytes, st)
    else:
      rc = lib.dt_flash_fwd_ex_noalloc(*common, nbytes, st)
    _lib.check(fn, rc)
    outs.append(o)
  torch.cuda.synchronize()
  assert torch.equal(outs[0], outs[1])
  rows = np.array([0, 777, 20000, s - 1])
  for bi, n in enumerate(lens):
    want = A.attention_f64(to64(q[bi, 1, rows])[None, None],
                           to64(k[bi, 1])[None, None],
                           to64(v[bi, 1])[None, None], kv_len=n)[0, 0]
    assert_attn_close(to64(outs[1][bi, 1, rows]), want, f"noalloc b{bi}")
