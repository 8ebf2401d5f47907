"""CPU-side checks of the C-ABI library: it loads and exports every symbol
the header declares, and argument validation fails with the documented codes
before anything touches a GPU."""
import ctypes
import re
from pathlib import Path

import pytest

from diffusers_tpu_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dt_attention.h"


def _declared():
  text = HEADER.read_text()
  text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
  return set(re.findall(r"\b(dt_[a-z0-9_]+)\s*\(", text))


def test_header_declares_bound_symbols():
  assert _declared() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
  lib = _lib.load()
  for name in _declared():
    assert hasattr(lib, name), name
  assert lib.dt_version() >= 300


def test_argument_errors_need_no_gpu():
  lib = _lib.load()
  s3 = _lib.i64_array(0, 0, 0)
  # null pointers
  rc = lib.dt_flash_fwd(None, None, None, None, 1, 1, 1, 1, 1, 128, s3, s3,
                        s3, s3, 0.0, 0, None, None, None, None, None)
  assert rc == _lib.DT_ERR_ARG
  assert b"null" in lib.dt_last_error()
  fake = ctypes.c_void_p(0x1000)
  st = _lib.i64_array(1024, 1024, 128)
  # unsupported head dim
  rc = lib.dt_flash_fwd(fake, fake, fake, fake, 1, 1, 1, 8, 8, 96, st, st, st,
                        st, 0.0, 0, None, None, None, None, None)
  assert rc == _lib.DT_ERR_UNSUPPORTED
  # GQA mismatch
  rc = lib.dt_flash_fwd(fake, fake, fake, fake, 1, 3, 2, 8, 8, 128, st, st, st,
                        st, 0.0, 0, None, None, None, None, None)
  assert rc == _lib.DT_ERR_SHAPE
  # kv_len beyond Skv
  rc = lib.dt_flash_fwd(fake, fake, fake, fake, 1, 1, 1, 8, 8, 128, st, st, st,
                        st, 0.0, 9, None, None, None, None, None)
  assert rc == _lib.DT_ERR_SHAPE
  # partial residual outputs
  rc = lib.dt_flash_fwd(fake, fake, fake, None, 1, 1, 1, 8, 8, 128, st, st, st,
                        st, 0.0, 0, None, fake, None, None, None)
  assert rc == _lib.DT_ERR_ARG
  w = ctypes.c_void_p(0x2000)
  dims = _lib.i32_array(44, 42, 40)  # rotate-half needs rotary/2 % 8 == 0
  rc = lib.dt_qk_norm_rope(fake, fake, fake, fake, 1, 4, 2, 128, st, st, w, w,
                           1e-6, None, _lib.ROPE_HALF, fake, dims, 1e4, -1,
                           None, None)
  assert rc == _lib.DT_ERR_UNSUPPORTED
  dims = _lib.i32_array(44, 43, 41)
  rc = lib.dt_qk_norm_rope(fake, fake, fake, fake, 1, 4, 2, 128, st, st, w, w,
                           1e-6, None, _lib.ROPE_PAIR, fake, dims, 1e4, -1,
                           None, None)
  assert rc == _lib.DT_ERR_ARG
  rc = lib.dt_qk_norm_rope(fake, fake, fake, fake, 1, 4, 2, 128, st, st, w, w,
                           1e-6, None, 7, fake, dims, 1e4, -1, None, None)
  assert rc == _lib.DT_ERR_ARG


def test_device_length_count_is_checked():
  """With a device length the host length argument is its entry count:
  0/1 (one for the batch) or B; anything else fails before any launch."""
  lib = _lib.load()
  fake = ctypes.c_void_p(0x1000)
  st = _lib.i64_array(1024, 1024, 128)
  for count, ok in ((3, False), (-1, False), (5, False)):
    rc = lib.dt_flash_fwd_ex(fake, fake, 0, fake, st, None, 0, fake, 2, 1, 1,
                             8, 8, 128, st, st, st, 0.0, count, fake, None,
                             None, None, None, None, None, None, 0, None)
    assert rc == _lib.DT_ERR_ARG, count
    assert b"entry count" in lib.dt_last_error()
  rc = lib.dt_pack_v(fake, fake, 2, 1, 64, 128, st, 3, fake, 1, None)
  assert rc == _lib.DT_ERR_ARG
  rc = lib.dt_smooth_keys(fake, fake, 2, 1, 64, 128, st, st, 7, fake, None,
                          fake, 1 << 20, None)
  assert rc == _lib.DT_ERR_ARG
  w = ctypes.c_void_p(0x2000)
  dims = _lib.i32_array(44, 42, 42)
  rc = lib.dt_qk_norm_rope(fake, fake, fake, fake, 2, 4, 2, 128, st, st, w, w,
                           1e-6, None, _lib.ROPE_HALF, fake, dims, 1e4, -1,
                           fake, None)
  assert rc == _lib.DT_ERR_ARG


def test_length_arg_host_forms():
  """Host-side length forms: per-sample sequences are range checked, equal
  values collapse to one host int, counts must match the batch."""
  import torch
  assert _lib.length_arg(None, 10, None) == (10, None)
  assert _lib.length_arg(7, 10, None) == (7, None)
  assert _lib.length_arg([7, 7], 10, None, batch=2) == (7, None)
  assert _lib.length_arg(torch.tensor([4, 4, 4]), 10, None, batch=3) == \
      (4, None)
  assert _lib.length_arg([9], 10, None, batch=2) == (9, None)
  import numpy as np
  assert _lib.length_arg(np.array([3, 3]), 10, None, batch=2) == (3, None)
  assert _lib.length_arg(np.int32(5), 10, None) == (5, None)
  with pytest.raises(ValueError):
    _lib.length_arg([7, 8, 9], 10, None, batch=2)    # wrong count
  with pytest.raises(ValueError):
    _lib.length_arg([7, 11], 10, None, batch=2)      # out of range
  with pytest.raises(ValueError):
    _lib.length_arg([0, 5], 10, None, batch=2)       # host 0 is refused
  with pytest.raises(ValueError):
    _lib.length_arg([7, 8], 10, None)                # no batch given
  with pytest.raises(ValueError):
    _lib.length_arg(torch.tensor([1.5]), 10, None)   # not an integer
  assert _lib.dev_count(torch.zeros(1)) == 0
  assert _lib.dev_count(torch.zeros(4)) == 4


def test_python_entry_rejects_cpu_tensors():
  import torch
  import diffusers_tpu_amd as dta
  x = torch.zeros(1, 1, 8, 64)
  with pytest.raises(ValueError, match="GPU"):
    dta.attention(x, x, x, scale=None, block_q=128, block_kv=128,
                  block_kv_compute=128)
  with pytest.raises(ValueError, match="GPU"):
    dta.qk_norm_rope(x, x, torch.ones(64), torch.ones(64))


def test_sdpa_configure_rejects_unknown_kernel():
  from diffusers_tpu_amd.kernels import mesh_attention
  with pytest.raises(ValueError):
    mesh_attention.configure(kernel="stock_splash")
  assert callable(mesh_attention.configure())


def test_residual_fixed_m_needs_mk():
  """kernels/splash.py:712-713: use_fixed_m without mk is a ValueError."""
  import torch
  import diffusers_tpu_amd as dta
  x = torch.zeros(1, 1, 8, 64)
  with pytest.raises(ValueError, match="mk"):
    dta.residual_attention(x, x, x, use_fixed_m=True)


def test_integration_stub_matches_the_binding():
  """The ctypes stub printed in INTEGRATION.md (section 2, plus the later
  blocks that add ``argtypes`` to it) binds the same symbols with the same
  signatures as ``_lib.SIGNATURES``: executed against a recorder in place of
  the library, every symbol it sets must carry the binding's restype and
  argtypes, and together they must cover every symbol."""
  text = (ROOT / "INTEGRATION.md").read_text()
  sec = text[text.index("## 2. The ctypes stub"):]
  blocks = [b.split("```")[0] for b in sec.split("```python")[1:]]
  blocks = blocks[:1] + [b for b in blocks[1:] if ".argtypes" in b]

  class Fn:
    restype = None
    argtypes = None

  class Lib:
    def __init__(self):
      self.fns = {}

    def __getattr__(self, name):
      return self.fns.setdefault(name, Fn())

  rec = Lib()
  real_cdll = ctypes.CDLL
  ctypes.CDLL = lambda *a, **k: rec
  env = {}
  try:
    for block in blocks:
      exec(compile(block, "INTEGRATION.md", "exec"), env)
  finally:
    ctypes.CDLL = real_cdll
  assert set(rec.fns) == set(_lib.SIGNATURES)
  for name, (res, args) in _lib.SIGNATURES.items():
    fn = rec.fns[name]
    assert fn.restype == res, name
    assert list(fn.argtypes or []) == list(args), name


def _prototypes():
  """name -> (return type, [parameter types]) of every prototype in the
  header, comments stripped."""
  text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
  text = re.sub(r"//[^\n]*", "", text)
  out = {}
  for m in re.finditer(r"([A-Za-z_][\w ]*?[\w*])\s*\b(dt_[a-z0-9_]+)\s*\(([^)]*)\)\s*;",
                       text):
    ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
    types = []
    if params and params != "void":
      for prm in params.split(","):
        prm = " ".join(prm.split())
        types.append(prm if "*" in prm else prm.rsplit(" ", 1)[0])
    out[name] = (ret, types)
  return out


def _ctype_of(c):
  c = c.replace("const ", "").strip()
  if "*" in c:
    return ctypes.c_char_p if c.startswith("char") else ctypes.c_void_p
  return {"int": ctypes.c_int, "float": ctypes.c_float,
          "size_t": ctypes.c_size_t, "int64_t": ctypes.c_int64}[c]


def test_binding_matches_the_header_prototypes():
  """Each ``_lib.SIGNATURES`` entry has the header prototype's arity and
  argument kinds (pointer / int / float / size_t / int64), so the ctypes
  binding cannot drift from the C declarations."""
  protos = _prototypes()
  assert set(protos) == set(_lib.SIGNATURES)
  for name, (res, args) in _lib.SIGNATURES.items():
    ret, params = protos[name]
    assert _ctype_of(ret) == res, (name, ret)
    assert [_ctype_of(p) for p in params] == list(args), name
