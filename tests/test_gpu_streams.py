"""Concurrent calls on separate streams: the entry points keep no mutable
global state (the static scratch of the no-allocation entry point aside),
so prologue + attention pipelines running at the same time on two streams,
each with its own workspace, give the bits each gives alone.  Host threads
drive the two streams, as a server with one stream per request would."""
import threading

import pytest
import torch

from gpu_helpers import banner, seeded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dta():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  import diffusers_tpu_amd
  return diffusers_tpu_amd


def _case(dta, seed, s, kv_len):
  q = seeded((1, s, 4, 128), seed)
  k = seeded((1, s, 4, 128), seed + 1)
  v = seeded((1, 4, s, 128), seed + 2)
  w = torch.ones(128)
  pos = torch.stack([torch.arange(s, dtype=torch.int32)] * 3, 1).cuda()
  rope = dta.RopeSpec("half", pos, (44, 42, 42), 1e4)

  def run(ws):
    qo, ko = dta.qk_norm_rope(q, k, w, w, rope=rope, valid_len=kv_len)
    return dta.attention(qo, ko, v, scale=None, block_q=256, block_kv=256,
                         block_kv_compute=256, kv_len=kv_len, workspace=ws)
  return run


def test_two_streams_concurrently(dta):
  banner("two streams, two host threads")
  cases = [_case(dta, 10, 40000, 39000), _case(dta, 20, 33333, None)]
  want = [c(dta.splash.AttentionWorkspace()) for c in cases]
  torch.cuda.synchronize()
  streams = [torch.cuda.Stream(), torch.cuda.Stream()]
  for s in streams:
    s.wait_stream(torch.cuda.current_stream())
  got = [[None] * 3, [None] * 3]
  errors = []

  def worker(i):
    try:
      ws = dta.splash.AttentionWorkspace()
      with torch.cuda.stream(streams[i]):
        for r in range(3):
          got[i][r] = cases[i](ws)
    except Exception as e:  # reported on the main thread
      errors.append(e)

  threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
  for t in threads:
    t.start()
  for t in threads:
    t.join()
  torch.cuda.synchronize()
  assert not errors, errors
  for i in range(2):
    for r in range(3):
      assert torch.equal(got[i][r], want[i]), (i, r)
