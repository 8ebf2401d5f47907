"""The hot path under HIP graph capture: prologue + attention captured once
and replayed several times, with eager work and synchronizations between the
replays, every replay checked against the eager result.  Neither entry point
allocates, synchronizes or writes memory through memset, so both capture."""
import pytest
import torch

from gpu_helpers import banner, seeded

pytestmark = pytest.mark.gpu


def test_prologue_and_attention_replay_in_a_graph():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd as dta
  banner("hip graph capture: prologue + attention")
  b, s, h, d = 1, 1000, 4, 128
  q = seeded((b, s, h, d), 150)
  k = seeded((b, s, h, d), 151)
  v = seeded((b, h, s, d), 152)
  wq = 1.0 + 0.02 * seeded((d,), 153, dtype=torch.float32)
  wk = 1.0 + 0.02 * seeded((d,), 154, dtype=torch.float32)
  pos = torch.stack([torch.zeros(s), torch.arange(s) // 40, torch.arange(s) % 40],
                    dim=1).to(torch.int32).cuda()
  rope = dta.RopeSpec("half", pos, (44, 42, 42), 1e4)
  qo = torch.empty((b, h, s, d), device="cuda", dtype=torch.bfloat16)
  ko = torch.empty_like(qo)
  out = torch.empty_like(qo)

  def step():
    dta.qk_norm_rope(q, k, wq, wk, eps=1e-6, rope=rope, valid_len=900,
                     out=(qo, ko))
    dta.splash._launch(qo, ko, v, None, 900, out=out)

  step()
  torch.cuda.synchronize()
  want = out.clone()
  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    step()                      # warm up on the capture stream
  torch.cuda.current_stream().wait_stream(side)
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    step()
  for r in range(4):
    out.zero_()                 # eager work between replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {r}"
