"""Size-independent properties of attention at the full sizes of the
workloads, where the float64 oracle can only check sampled rows:

* linearity in V: doubling V doubles o bit for bit (a power-of-two scale
  commutes with every rounding);
* padding independence: keys at or past kv_len never matter, whatever they
  hold (bit-identical);
* a constant added to every value row adds itself to o (the probabilities
  sum to one);
* the LSE merge of the residuals of two key halves equals the whole call;
* reversing the key order (K and V together) leaves o unchanged up to the
  accumulation order.
"""
import pytest
import torch

from gpu_helpers import ATTN_MAX_ABS, ATTN_MEAN_ABS, banner

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _close(got, want, what):
  err = (got.float() - want.float()).abs()
  assert torch.isfinite(got.float()).all(), what
  assert err.max().item() <= ATTN_MAX_ABS, (what, err.max().item())
  assert err.mean().item() <= ATTN_MEAN_ABS, (what, err.mean().item())


@pytest.mark.parametrize("name", ["I1", "V4", "V7"])
def test_full_size_properties(dta, name):
  from diffusers_tpu_amd.workloads import WORKLOADS
  w = WORKLOADS[name]
  banner(f"properties {name} B={w.B} H={w.H} S={w.S} kv_len={w.kv_len}")
  g = torch.Generator(device="cuda").manual_seed(11)
  shape = (w.B, w.H, w.S, w.D)
  q = torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=g)
  k = torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=g)
  v = torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=g)
  n = w.kv_len
  kw = dict(scale=None, block_q=2048, block_kv=2048, block_kv_compute=512)
  ws = dta.splash.AttentionWorkspace()
  att = lambda q_, k_, v_, **x: dta.attention(q_, k_, v_, kv_len=n,
                                              workspace=ws, **kw, **x)
  o = att(q, k, v)
  # linearity in V
  assert torch.equal(att(q, k, v * 2), o * 2)
  # padding independence (only where the workload pads)
  if n < w.S:
    k2, v2 = k.clone(), v.clone()
    k2[:, :, n:] = 1e4
    v2[:, :, n:] = float("nan")
    assert torch.equal(att(q, k2, v2), o)
    del k2, v2
  # a constant value row shifts o by itself
  u = torch.randn((1, 1, 1, w.D), device="cuda", generator=g).to(torch.bfloat16)
  _close(att(q, k, v + u), (o.float() + u.float()), f"{name} shift")
  # LSE merge of two key halves (residual form) equals the whole call
  half = (n // 2 // 64) * 64
  o1, m1, l1 = dta.residual_attention(q, k[:, :, :half], v[:, :, :half], **kw)
  o2, m2, l2 = dta.residual_attention(q, k[:, :, half:n], v[:, :, half:n], **kw)
  merged = dta.splash.merge_residuals([(o1, m1, l1), (o2, m2, l2)])
  _close(merged, o, f"{name} merge")
  del o1, o2, merged
  # key order reversed (K and V rows together)
  rev = torch.arange(n - 1, -1, -1, device="cuda")
  kr = k[:, :, :n].index_select(2, rev)
  vr = v[:, :, :n].index_select(2, rev)
  _close(dta.attention(q, kr, vr, **kw), o, f"{name} reversed keys")
  torch.cuda.synchronize()


@pytest.mark.parametrize("name", ["I1", "V7"])
def test_full_size_prologue_row_norms(dta, name):
  """Every row of the prologue at full size: with unit RMSNorm weights the
  rotation keeps each row's RMS at 1 (the oracle checks sampled rows;
  this covers all of them), and rows at or past the valid length are
  zero."""
  from diffusers_tpu_amd.workloads import WORKLOADS
  w = WORKLOADS[name]
  banner(f"prologue norms {name} B={w.B} H={w.H} S={w.S}")
  x = w.inputs(device="cuda")
  ones = torch.ones(w.D)
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  vl = w.kv_len if w.padded else None
  qo, ko = dta.qk_norm_rope(x["q"], x["k"], ones, ones, eps=w.eps, rope=rope,
                            valid_len=vl)
  n = w.kv_len if w.padded else w.S
  for t in (qo, ko):
    rms = t[:, :, :n].float().pow(2).mean(-1).sqrt()
    assert (rms - 1).abs().max().item() < 1e-2, name
    if n < w.S:
      assert torch.all(t[:, :, n:] == 0)
