"""The five BASELINE workloads at full size through the whole path
(prologue -> attention), checked against the float64 oracle on sampled rows.

RMSNorm + RoPE is row-local, so sampled token rows of the prologue output are
compared with the oracle applied to the same input rows.  Attention is
checked on sampled query rows of two heads against the oracle run over the
full key range (the kernel's own prologue output as q/k, so the attention
check does not re-count prologue rounding).
"""
import numpy as np
import pytest
import torch

from gpu_helpers import (assert_attn_close, assert_prologue_close, banner,
                         to64)
from oracle import attention as A
from oracle import norm_rope as NR

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _sample_rows(w, n, rng):
  rows = set(rng.choice(w.S, size=n, replace=False).tolist())
  rows |= {0, w.S - 1, w.kv_len - 1}
  if w.padded:
    rows |= {w.kv_len, min(w.S - 1, w.kv_len + 1)}
  return np.array(sorted(rows))


@pytest.mark.parametrize("name", ["P", "I1", "I2", "V4", "V7"])
def test_workload_end_to_end(dta, name):
  from diffusers_tpu_amd.workloads import WORKLOADS
  w = WORKLOADS[name]
  banner(f"workload {name} S={w.S} H={w.H} D={w.D} kv_len={w.kv_len}")
  x = w.inputs(device="cuda")
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  qa, ka = dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps,
                            rope=rope, q_head_scale=x["hs"],
                            valid_len=w.kv_len if w.padded else None)
  v = x["v"].to(torch.bfloat16)
  out = dta.attention(qa, ka, v, scale=None, block_q=2048, block_kv=2048,
                      block_kv_compute=512,
                      kv_len=w.kv_len if w.padded else None)
  torch.cuda.synchronize()
  assert out.shape == (w.B, w.H, w.S, w.D)
  assert out.dtype == torch.bfloat16
  rng = np.random.default_rng(7)
  rows = _sample_rows(w, 48, rng)
  pos = w.positions()[rows]
  hs = None if x["hs"] is None else x["hs"].cpu().numpy()
  # --- prologue on sampled rows
  for src, wt, got, is_q in ((x["q"], x["wq"], qa, True),
                             (x["k"], x["wk"], ka, False)):
    inp = to64(src[:, rows])                          # (B, r, H, D)
    want = NR.qk_norm_rope_f64(inp, wt.cpu().numpy(), w.eps, pos,
                               w.axis_dims, w.theta, w.mode,
                               head_scale=hs if is_q else None)
    if w.padded:
      want[:, rows >= w.kv_len] = 0
    g = to64(got[:, :, rows].transpose(1, 2))
    e = assert_prologue_close(g, want, f"{name} prologue")
    print(f"{name} prologue: arithmetic error {e['kernel']:.3g}, "
          f"{e['exact']:.5f} correctly rounded, max {e['steps']:.0f} bf16 "
          f"step, vs f64 {e['full']:.3g}", flush=True)
  # --- attention on sampled query rows of two heads
  for b in range(w.B):
    for h in sorted({0, w.H - 1}):
      q64 = to64(qa[b, h, rows])[None, None]
      k64 = to64(ka[b, h])[None, None]
      v64 = to64(v[b, h])[None, None]
      want = A.attention_f64(q64, k64, v64, kv_len=w.kv_len)[0, 0]
      got = to64(out[b, h, rows])
      assert_attn_close(got, want, f"{name} b{b} h{h}")
  assert torch.isfinite(out.float()).all()
