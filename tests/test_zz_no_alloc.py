"""dt_flash_fwd_ex_noalloc (the tail split's workspace in the library's
static device scratch) against dt_flash_fwd_ex with a caller workspace of
the same size, through the C ABI: two calls in a row, the second smaller,
bit-equal (same split plan, same kernels)."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_attn_close, banner, seeded, to64
from oracle import attention as A

pytestmark = pytest.mark.gpu


def _call(lib, fn, q, k, v, vt, tiles, o, kv_len, nbytes, ws=None):
  from diffusers_tpu_amd import _lib
  s3 = lambda t: _lib.i64_array(*t.stride()[:3])
  b, hq, sq, d = q.shape
  _, hkv, skv, _ = k.shape
  st = torch.cuda.current_stream().cuda_stream
  vargs = ((None, None, vt.data_ptr(), tiles) if vt is not None
           else (v.data_ptr(), s3(v), None, 0))
  common = (q.data_ptr(), k.data_ptr(), 0, *vargs, o.data_ptr(), b, hq, hkv,
            sq, skv, d, s3(q), s3(k), s3(o), 1.0 / d ** 0.5, kv_len, None,
            None, None, None, None, None, None)
  if fn == "noalloc":
    return lib.dt_flash_fwd_ex_noalloc(*common, nbytes, st)
  return lib.dt_flash_fwd_ex(*common, None if ws is None else ws.data_ptr(),
                             nbytes, st)


def test_noalloc_matches_workspace_entry():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd import _lib
  from diffusers_tpu_amd.kernels import splash as sp
  lib = _lib.load()
  cap = _lib.NOALLOC_SCRATCH_BYTES
  cases = [  # (B, H, S, kv_len, packed V): the second call is the smaller
      (1, 2, 40000, 39000, True),
      (1, 3, 5000, 4321, False),
  ]
  for i, (b, h, s, n, packed) in enumerate(cases):
    banner(f"noalloc call {i}: B{b} H{h} S{s} kv_len {n} packed={packed}")
    q = seeded((b, h, s, 128), 400 + i)
    k = seeded((b, h, s, 128), 410 + i)
    v = seeded((b, h, s, 128), 420 + i)
    vt, tiles = sp.pack_v(v, n) if packed else (None, 0)
    need = lib.dt_flash_fwd_workspace_bytes(b, h, s, s, n, 128)
    assert need > 0, "the case should take the tail split"
    nbytes = min(need, cap)
    ws = torch.empty((nbytes + 3) // 4, device="cuda", dtype=torch.float32)
    want = torch.empty_like(q)
    got = torch.full_like(q, float("nan"))
    _lib.check("dt_flash_fwd_ex",
               _call(lib, "ex", q, k, v, vt, tiles, want, n, nbytes, ws))
    _lib.check("dt_flash_fwd_ex_noalloc",
               _call(lib, "noalloc", q, k, v, vt, tiles, got, n, nbytes))
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"call {i}: differs from dt_flash_fwd_ex"
    # and the oracle on sampled rows (the merged split rows included)
    rows = np.array([0, 1, s // 2, s - 257, s - 1])
    for hh in (0, h - 1):
      ref = A.attention_f64(to64(q[0, hh, rows])[None, None],
                            to64(k[0, hh])[None, None],
                            to64(v[0, hh])[None, None], kv_len=n)[0, 0]
      assert_attn_close(to64(got[0, hh, rows]), ref, f"noalloc call {i}")
    # no split: scratch_bytes 0 equals the workspace-free call
    got0 = torch.empty_like(q)
    want0 = torch.empty_like(q)
    _lib.check("dt_flash_fwd_ex_noalloc",
               _call(lib, "noalloc", q, k, v, vt, tiles, got0, n, 0))
    _lib.check("dt_flash_fwd_ex",
               _call(lib, "ex", q, k, v, vt, tiles, want0, n, 0))
    torch.cuda.synchronize()
    assert torch.equal(got0, want0)


def test_noalloc_rejects_oversized_scratch():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  from diffusers_tpu_amd import _lib
  lib = _lib.load()
  q = seeded((1, 1, 256, 128), 430)
  o = torch.empty_like(q)
  rc = _call(lib, "noalloc", q, q, q, None, 0, o, 0,
             _lib.NOALLOC_SCRATCH_BYTES + 16)
  assert rc == _lib.DT_ERR_ARG
  assert b"scratch" in lib.dt_last_error()
