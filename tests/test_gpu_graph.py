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


def _replay_check(step, out, tries=4):
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
  for r in range(tries):
    out.zero_()                 # eager work between replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {r}"


def test_packed_v_and_split_replay_in_a_graph():
  """The V pack, the split attention kernel and its merge launch in one
  graph (S above the packed-V threshold, 157 query blocks: split)."""
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd as dta
  banner("hip graph capture: packed V + tail split")
  s = 40000
  assert s >= dta.splash.PACKED_V_MIN_KEYS
  q = seeded((1, 1, s, 128), 155)
  k = seeded((1, 1, s, 128), 156)
  v = seeded((1, 1, s, 128), 157)
  out = torch.empty_like(q)
  _replay_check(lambda: dta.splash._launch(q, k, v, None, 39000, out=out), out)


def test_fixed_m_dispatch_replay_in_a_graph():
  """The dispatch op's k-smoothing, fixed-m bound and attention in one
  graph (torch fills, no memset)."""
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  banner("hip graph capture: fixed-m dispatch op")
  from diffusers_tpu_amd.backends import splash_dispatch  # registers the op
  del splash_dispatch
  q = seeded((1, 3, 700, 128), 158)
  k = seeded((1, 3, 700, 128), 159)
  v = seeded((1, 3, 700, 128), 160)
  out = torch.empty_like(q)
  def step():
    out.copy_(torch.ops.dt.splash_attention(q, k, v, True, False, True))
  _replay_check(step, out)
