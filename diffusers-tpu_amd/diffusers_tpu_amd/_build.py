"""Builds libdt_attention.so for gfx950 with hipcc (no torch extension).

The library is a plain C-ABI shared object (``include/dt_attention.h``); it
is built in-tree next to this file so that it travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
PROJECT_DIR = PKG_DIR.parent
CSRC = PROJECT_DIR / "csrc"
LIB_NAME = "libdt_attention.so"
LIB_PATH = PKG_DIR / LIB_NAME
# bench.py's HBM calibration copy (not part of the attention path's ABI)
CALIB_SOURCES = ["calib/hbm_copy.hip"]
CALIB_PATH = PKG_DIR / "libdt_calib.so"

SOURCES = ["capi.cpp", "qk_norm_rope.hip", "flash_fwd.hip", "flash_attn.hip",
           "flash_wide.hip",
           "row_norm.hip", "fp8_cast.hip", "v_pack.hip",
           "k_smooth.hip"]
ARCH = "gfx950"
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Keep the compiler away from packed-fp32 VALU forms.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
  rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
  return str(Path(rocm) / "bin" / "hipcc")


def build(verbose: bool = False, jobs: int = 4) -> Path:
  """Compiles every source (in parallel) and links the shared libraries:
  the attention path's, and the benchmark's calibration copy."""
  _build_lib(SOURCES, LIB_PATH, verbose, jobs)
  _build_lib(CALIB_SOURCES, CALIB_PATH, verbose, jobs)
  return LIB_PATH


def _build_lib(sources, lib_path, verbose, jobs):
  obj_dir = PROJECT_DIR / "_build"
  obj_dir.mkdir(exist_ok=True)
  procs = []
  objs = []
  for src in sources:
    obj = obj_dir / (Path(src).stem + ".o")
    objs.append(obj)
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(PROJECT_DIR.parent / "include"),
           "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
      print(" ".join(cmd), flush=True)
    procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                        stderr=subprocess.STDOUT)))
    if len(procs) >= jobs:
      _wait(procs.pop(0))
  for pr in procs:
    _wait(pr)
  tmp = lib_path.with_suffix(".so.tmp")
  cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}",
         *[str(o) for o in objs], "-o", str(tmp)]
  out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
  if out.returncode:
    raise RuntimeError(f"link failed:\n{out.stdout}")
  os.replace(tmp, lib_path)


def _wait(item):
  src, proc = item
  out, _ = proc.communicate()
  text = out.decode(errors="replace")
  lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
  if proc.returncode:
    raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(lines))


if __name__ == "__main__":
  print(build(verbose="-v" in sys.argv))
