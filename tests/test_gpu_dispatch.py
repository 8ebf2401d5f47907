"""The diffusers dispatch replacement with the real op on the GPU
(backends/ours_splash_tt.py:92-157), eagerly and under torch.compile."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sd():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd.backends import splash_dispatch
  return splash_dispatch


def _fallback(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=False, **kw):
  raise AssertionError("fallback taken")


@pytest.mark.parametrize("fixed_m", [False, True])
def test_dispatch_matches_oracle(sd, fixed_m):
  banner(f"dispatch fixed_m={fixed_m}")
  d = sd.make_dispatch(_fallback, fixed_m=fixed_m, min_seq=256)
  q = seeded((1, 600, 4, 128), 140)       # diffusers layout (B, S, H, D)
  k = seeded((1, 600, 4, 128), 141)
  v = seeded((1, 600, 4, 128), 142)
  out = d(q, k, v)
  torch.cuda.synchronize()
  assert out.shape == q.shape
  want = A.attention_f64(*(to64(t.transpose(1, 2)) for t in (q, k, v)))
  assert_attn_close(to64(out.transpose(1, 2)), want, "dispatch")


def test_dispatch_under_torch_compile(sd):
  banner("dispatch under torch.compile(backend=aot_eager)")
  d = sd.make_dispatch(_fallback, fixed_m=True, min_seq=256)
  q = seeded((1, 512, 2, 128), 143)
  k = seeded((1, 512, 2, 128), 144)
  v = seeded((1, 512, 2, 128), 145)
  f = torch.compile(lambda a, b, c: d(a, b, c) * 2.0, backend="aot_eager",
                    fullgraph=True)
  got = f(q, k, v)
  ref = d(q, k, v) * 2.0
  torch.cuda.synchronize()
  assert torch.equal(got, ref)


@pytest.mark.parametrize("fused,fixed_m", [(False, True), (True, False)])
def test_bhsd_processor_matches_oracle(sd, fused, fixed_m):
  """BHSD-first processor (ours_splash_tt.py:165-231): projections in
  torch, norm + RoPE from H3's (cos, sin) tables in the fused prologue,
  attention, output projection.  The attention output (before to_out) is
  checked against the float64 composition of the reference's steps on the
  same projected q, k, v; to_out is then the module's own projection."""
  from oracle import norm_rope as NR
  from test_dispatch import _Attn
  banner(f"bhsd processor fused={fused} fixed_m={fixed_m}")
  torch.manual_seed(150)
  h, d, s = 4, 128, 600
  attn = _Attn(h * d, h, eps=1e-5, fused=fused).to("cuda", torch.bfloat16)
  with torch.no_grad():
    attn.norm_q.weight.copy_(1 + 0.05 * torch.randn(d))
    attn.norm_k.weight.copy_(1 + 0.05 * torch.randn(d))
  hs = seeded((1, s, h * d), 151)
  ang = torch.rand(s, 48, dtype=torch.float64) * 40
  cos = torch.cos(torch.cat([ang, ang], -1)).float().cuda()
  sin = torch.sin(torch.cat([ang, ang], -1)).float().cuda()
  def orig(*a, **k):
    raise AssertionError("original processor reached")
  call = sd.make_processor_call(
      orig, sd.make_dispatch(_fallback, fixed_m=fixed_m, min_seq=256),
      min_seq=256)
  with torch.no_grad():
    out = call(None, attn, hs, rotary_emb=(cos, sin))
    to_out = attn.to_out
    attn.to_out = torch.nn.ModuleList([torch.nn.Identity(),
                                       torch.nn.Identity()])
    mid = call(None, attn, hs, rotary_emb=(cos, sin))
    attn.to_out = to_out
    if fused:
      q, k, v = attn.to_qkv(hs).chunk(3, dim=-1)
    else:
      q, k, v = attn.to_q(hs), attn.to_k(hs), attn.to_v(hs)
    proj = to_out[0](mid)
  torch.cuda.synchronize()
  assert out.shape == hs.shape and torch.equal(out, proj)
  q, k, v = (to64(t.unflatten(-1, (h, d))) for t in (q, k, v))
  c64, s64 = cos.double().cpu().numpy(), sin.double().cpu().numpy()
  wq = to64(attn.norm_q.weight)
  wk = to64(attn.norm_k.weight)
  qr = NR.h3_apply_rope_f64(NR.rms_norm_f64(q, wq, 1e-5), c64, s64)
  kr = NR.h3_apply_rope_f64(NR.rms_norm_f64(k, wk, 1e-5), c64, s64)
  want = A.attention_f64(*(x.transpose(0, 2, 1, 3) for x in (qr, kr, v)))
  want = want.transpose(0, 2, 1, 3).reshape(1, s, h * d)
  assert_attn_close(to64(mid), want, "bhsd processor")
