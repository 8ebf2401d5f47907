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
