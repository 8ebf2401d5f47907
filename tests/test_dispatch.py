"""The diffusers dispatch replacement (backends/ours_splash_tt.py:92-157):
routing, layout and k-smoothing, on the CPU with a stand-in kernel; the real
op runs in tests/test_gpu_dispatch.py."""
import pytest
import torch

from diffusers_tpu_amd.backends import splash_dispatch as SD


def _sdpa_bhsd(q, k, v):
  return torch.nn.functional.scaled_dot_product_attention(q, k, v)


def test_routes_and_falls_back():
  calls = []
  def original(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=False, **kw):
    calls.append((tuple(q.shape), attn_mask is not None, is_causal, dropout_p))
    return torch.zeros_like(q)
  seen = []
  def kernel(q, k, v):
    seen.append((tuple(q.shape), float(k.mean(dim=-2).abs().max())))
    return _sdpa_bhsd(q, k, v)
  d = SD.make_dispatch(original, op=kernel, min_seq=64)
  q = torch.randn(1, 80, 2, 16)          # (B, S, H, D)
  k = torch.randn(1, 80, 2, 16) + 3.0
  v = torch.randn(1, 80, 2, 16)
  out = d(q, k, v)
  assert out.shape == q.shape and len(seen) == 1 and not calls
  assert seen[0][0] == (1, 2, 80, 16)    # the kernel saw (B, H, S, D)
  assert seen[0][1] < 1e-5               # keys were k-smoothed
  # k-smoothing does not change softmax attention
  want = _sdpa_bhsd(q.transpose(1, 2), k.transpose(1, 2),
                    v.transpose(1, 2)).transpose(1, 2)
  torch.testing.assert_close(out, want, atol=1e-5, rtol=1e-5)
  # mask / causal / dropout / short sequences go to the original
  d(q, k, v, attn_mask=torch.ones(80, 80, dtype=torch.bool))
  d(q, k, v, is_causal=True)
  d(q, k, v, dropout_p=0.1)
  d(q[:, :10], k[:, :10], v[:, :10])
  assert len(calls) == 4 and len(seen) == 1
  assert d.stats == {"n": 1, "fallback": 4}
  # already-(B,H,S,D) callers get diffusers' (B,S,H,D) back, as from the
  # fallback, whose inputs are transposed to that layout
  out2 = d(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
           _already_bhsd=True)
  torch.testing.assert_close(out2, want, atol=1e-5, rtol=1e-5)
  d(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True,
    _already_bhsd=True)
  assert calls[-1][0] == (1, 80, 2, 16)


def test_install_without_diffusers_reports_false():
  msgs = []
  assert SD.install(verbose=msgs.append) in (True, False)
  try:
    import diffusers  # noqa: F401
  except ImportError:
    assert msgs and "diffusers" in msgs[0]


def test_op_is_registered_with_a_fake():
  from torch._subclasses.fake_tensor import FakeTensorMode
  with FakeTensorMode():
    q = torch.empty(1, 2, 300, 128, dtype=torch.bfloat16)
    out = torch.ops.dt.splash_attention(q, q, q, True, False)
    assert out.shape == q.shape and out.dtype == q.dtype


class _Attn(torch.nn.Module):
  """The attributes the BHSD-first processor reads from diffusers'
  ``Attention`` module (ours_splash_tt.py:172-228)."""

  def __init__(self, dim, heads, eps=1e-5, fused=False, norm=torch.nn.RMSNorm):
    super().__init__()
    self.heads = heads
    self.fused_projections = fused
    d = dim // heads
    if fused:
      self.to_qkv = torch.nn.Linear(dim, 3 * dim, bias=False)
    else:
      self.to_q = torch.nn.Linear(dim, dim, bias=False)
      self.to_k = torch.nn.Linear(dim, dim, bias=False)
      self.to_v = torch.nn.Linear(dim, dim, bias=False)
    self.norm_q = norm(d, eps=eps)
    self.norm_k = norm(d, eps=eps)
    self.to_out = torch.nn.ModuleList([torch.nn.Linear(dim, dim),
                                       torch.nn.Dropout(0.0)])


def test_processor_falls_back_to_the_original():
  """Masked calls, short sequences and non-RMSNorm norms keep the
  processor it replaces; none of them reaches the kernels (CPU)."""
  seen = []
  def orig(self, attn, hs, rotary_emb=None, attention_mask=None):
    seen.append(attention_mask is not None)
    return hs
  def no_dispatch(*a, **k):
    raise AssertionError("dispatch reached")
  call = SD.make_processor_call(orig, no_dispatch, min_seq=64)
  attn = _Attn(64, 2)
  hs = torch.randn(1, 100, 64)
  call(None, attn, hs, attention_mask=torch.ones(100, 100, dtype=torch.bool))
  call(None, attn, hs[:, :10])
  call(None, _Attn(64, 2, norm=lambda d, eps: torch.nn.LayerNorm(d, eps=eps)),
       hs)
  odd = _Attn(64, 2)
  odd.norm_k.eps = 1e-6
  call(None, odd, hs)
  # H3's test_block shape (jax_dit.py:818-880): 4 heads of 32 channels
  call(None, _Attn(128, 4), torch.randn(1, 100, 128))
  assert seen == [True, False, False, False, False]


def test_halves_cache_answers_only_for_the_same_tables(monkeypatch):
  """The halves check is cached per tensor object and version: a new
  tensor (even at a reused address) or an in-place update is checked
  again (CPU; the check itself is stubbed to count calls)."""
  from diffusers_tpu_amd.kernels import qk_norm_rope as QNR
  calls = []

  def fake_check(cos, sin):
    calls.append(1)
    return bool((cos[..., : cos.shape[-1] // 2] ==
                 cos[..., cos.shape[-1] // 2:]).all())
  monkeypatch.setattr(QNR, "check_halves", fake_check)
  cache = SD._HalvesCache()
  cos = torch.ones(8, 4)
  sin = torch.zeros(8, 4)
  assert cache(cos, sin) and cache(cos, sin)
  assert len(calls) == 1
  cos[:, 3] = 2.0                 # in-place: halves now differ
  assert not cache(cos, sin)
  assert len(calls) == 2
  other = torch.ones(8, 4)
  other[:, 0] = 5.0               # a different tensor with differing halves
  assert not cache(other, sin)
  assert len(calls) == 3
  del cos, other
  for _ in range(4):              # new tensors, some at reused addresses
    c = torch.ones(8, 4)
    c[:, 1] = 3.0
    assert not cache(c, sin)
  assert len(calls) == 7
