"""Tensors past 2^31 elements: every offset the kernels form from (batch,
head, row) must be 64-bit.  One call each of the prologue, the attention
kernel (row-major and packed V) and the E4M3 key cast over 32,769 heads of
512 rows x 128 channels (2.15e9 elements per tensor), checked on heads
whose data lies past element 2^31 against the float64 oracle."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, assert_prologue_close, banner, to64
from oracle import attention as A
from oracle import fp8 as P8
from oracle import norm_rope as NR

pytestmark = pytest.mark.gpu

H, S, D = 32769, 512, 128   # H * S * D = 2^31 + 65536
CHECK = [0, H - 2, H - 1]   # one head below 2^31 elements, two past it


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _randn(shape, seed):
  g = torch.Generator(device="cuda").manual_seed(seed)
  return torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=g)


def test_attention_past_2_31_elements(dta):
  banner(f"large index attention H={H} S={S} D={D}")
  assert H * S * D > 2**31
  q = _randn((1, H, S, D), 1)
  k = _randn((1, H, S, D), 2)
  v = _randn((1, H, S, D), 3)
  kw = dict(scale=None, block_q=256, block_kv=256, block_kv_compute=256)
  o = dta.attention(q, k, v, **kw)
  # packed V, as the kernel streams it from 32768 keys on
  from diffusers_tpu_amd.kernels import splash
  vt = splash.pack_v(v)
  o_packed = splash._launch(q, k, v, None, None, packed_v=vt)
  torch.cuda.synchronize()
  assert torch.equal(o, o_packed)
  for h in CHECK:
    want = A.attention_f64(to64(q[:, h:h + 1]), to64(k[:, h:h + 1]),
                           to64(v[:, h:h + 1]))
    assert_attn_close(to64(o[:, h:h + 1]), want, f"head {h}")
  del o, o_packed, vt
  # E4M3 keys: the cast kernel and the E4M3 product at the same extents
  o8 = dta.attention(q, k, v, qk_fp8=True, **kw)
  torch.cuda.synchronize()
  c = np.log2(np.e) / np.sqrt(D)
  for h in CHECK:
    q8 = P8.e4m3_round(to64((q[:, h:h + 1].float() * c).to(torch.bfloat16)))
    k8 = P8.e4m3_round(to64(k[:, h:h + 1]))
    want8 = A.attention_f64(q8, k8, to64(v[:, h:h + 1]), scale=np.log(2.0))
    assert_attn_close(to64(o8[:, h:h + 1]), want8, f"qk_fp8 head {h}")


def test_prologue_past_2_31_elements(dta):
  banner(f"large index prologue S={S} H={H} D={D}")
  q = _randn((1, S, H, D), 4)
  k = _randn((1, S, H, D), 5)
  wq = torch.ones(D)
  wk = torch.ones(D)
  pos = torch.stack([torch.arange(S, dtype=torch.int32)] * 3, 1) % 64
  rope = dta.RopeSpec("half", pos.cuda(), (44, 42, 42), 1e4)
  qo, ko = dta.qk_norm_rope(q, k, wq, wk, eps=1e-6, rope=rope)
  torch.cuda.synchronize()
  for h in CHECK:
    for x, out in ((q, qo), (k, ko)):
      want = NR.qk_norm_rope_f64(to64(x[:, :, h:h + 1]), np.ones(D), 1e-6,
                                 pos.numpy(), (44, 42, 42), 1e4, "half")
      assert_prologue_close(to64(out[:, h:h + 1].transpose(1, 2)), want,
                            f"head {h}")
