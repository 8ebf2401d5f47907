"""Benchmark of the DiT attention hot path on one MI355X.

A step is one attention layer's hot path on the 350,784-token video head
shard ("V7": B=1, H=5 of 40, S=350,784, D=128, bf16):
the fused QK-RMSNorm + 3D-RoPE prologue on q and k, then the non-causal
flash-attention forward.  Inputs are seeded synthetic tensors resident in HBM
before the timed region.

Prints ONE JSON line.  `value` is attention TFLOP/s over the whole step
(4*B*H*Sq*Skv_valid*D / step time); `roofline` is the flash kernel's
MFMA-bound roofline from its own HIP-event-timed launches; `prologue` the
prologue kernel's HBM roofline; `cpu_baseline` the torch-CPU float32 port of
the reference's CPU attention path on a bounded sample of query rows.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "diffusers-tpu_amd")):
  if _p not in sys.path:
    sys.path.insert(0, _p)

METRIC = ("attention TFLOP/s + % bf16 MFMA peak at 350,784-token video shard; "
          "ms/layer")


def _traffic(kernel: str, workload: str):
  """HBM bytes per launch measured with rocprofv3 --pmc (profiles/)."""
  path = os.path.join(ROOT, "profiles", "traffic.json")
  try:
    with open(path) as f:
      return json.load(f).get(workload, {}).get(kernel)
  except (OSError, ValueError):
    return None


def cpu_baseline(w, x_cpu, target_s=12.0):
  """torch-CPU fp32 attention (the oracle's CPU leg) on sampled query rows.

  Times R query rows of head 0 against all valid keys and extrapolates to
  TFLOP/s (attention work is linear in query rows, so the rate of a row
  sample is the rate of the whole call).  R is sized from a short probe so
  the sample takes about `target_s` seconds.  Threads: every core this
  process may run on (its affinity set), unless OMP_NUM_THREADS sets the
  job's CPU share lower; both numbers are reported.
  """
  import torch
  from oracle import attention as A
  visible = len(os.sched_getaffinity(0))
  share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
  threads = min(visible, share) if share > 0 else visible
  torch.set_num_threads(threads)
  q, k, v = x_cpu
  n = w.kv_len

  def run(rows):
    t0 = time.perf_counter()
    for r0 in range(0, rows, 512):
      r1 = min(rows, r0 + 512)
      A.attention_torch_f32(q[:, :1, r0:r1], k[:, :1], v[:, :1], kv_len=n)
    return time.perf_counter() - t0

  probe_rows = 256
  t_probe = run(probe_rows)
  rows = int(min(w.S, max(probe_rows, probe_rows * target_s / t_probe)))
  rows = max(probe_rows, rows // 256 * 256)
  t = run(rows)
  flops = 4.0 * rows * n * w.D
  sampled = rows / (w.B * w.H * w.S)
  rate = flops / t
  return {"value": rate / 1e12, "unit": "TFLOP/s", "cores": threads,
          "host_cores_visible": visible,
          "omp_num_threads": share or None,
          "kind": "port", "extrapolated": True,
          "sampled_fraction": round(sampled, 6),
          "full_call_s_extrapolated": round(w.attn_flops() / rate, 1),
          "sample": f"{rows} query rows x {n} keys x D={w.D}, head 0 of "
                    f"{w.name} ({100 * sampled:.2f} % of the call's query "
                    f"rows, timed {t:.1f} s and extrapolated linearly in "
                    f"rows); torch-CPU fp32 SDPA on {threads} threads"}


def _steady(fn, torch, warm_s, timed_s):
  """(ms per call, calls timed) of fn in steady state: back to back for
  about warm_s seconds first, then HIP events over about timed_s."""
  fn()
  torch.cuda.synchronize()
  t0 = time.perf_counter()
  n_warm = 0
  while time.perf_counter() - t0 < warm_s:
    fn()
    n_warm += 1
    if n_warm % 8 == 0:
      torch.cuda.synchronize()
  torch.cuda.synchronize()
  per = (time.perf_counter() - t0) / n_warm
  reps = int(min(2000, max(5, timed_s / per)))
  e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
  e0.record()
  for _ in range(reps):
    fn()
  e1.record()
  torch.cuda.synchronize()
  return round(e0.elapsed_time(e1) / reps, 4), reps


def cfg_pair(dta, torch, lens=(4396, 4233), warm_s=0.3, timed_s=0.2):
  """I1's CFG pair with per-sample key lengths (the two prompts' real text
  differs: 300 and 137 of 512 rows): the attention call with a device
  int32[2] length, one launch over both samples, against the reference's
  form, one B=1 call per sample (models/moss_image/jax_dit.py:198-202)."""
  from diffusers_tpu_amd.workloads import MFMA_BF16_DENSE_PEAK, WORKLOADS
  w = WORKLOADS["I1"]
  x = w.inputs(device="cuda")
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  n_dev = torch.tensor(lens, device="cuda", dtype=torch.int32)
  qo, ko = dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps,
                            rope=rope, valid_len=n_dev)
  v = x["v"].to(torch.bfloat16).clone()
  for b, n in enumerate(lens):
    v[b, :, n:] = 0
  out = torch.empty_like(qo)
  ws = dta.splash.AttentionWorkspace()
  ws1 = dta.splash.AttentionWorkspace()
  one = lambda: dta.attention(qo, ko, v, kv_len=n_dev, out=out, workspace=ws)
  def loop():
    for b, n in enumerate(lens):
      dta.attention(qo[b:b + 1], ko[b:b + 1], v[b:b + 1], kv_len=n,
                    out=out[b:b + 1], workspace=ws1)
  flops = sum(4.0 * w.H * w.S * n * w.D for n in lens)
  ms1, _ = _steady(one, torch, warm_s, timed_s)
  ms2, _ = _steady(loop, torch, warm_s, timed_s)
  return {"lengths": list(lens), "one_launch_ms": ms1,
          "one_launch_frac": round(flops / (ms1 * 1e-3) / MFMA_BF16_DENSE_PEAK, 4),
          "per_sample_calls_ms": ms2,
          "per_sample_calls_frac": round(flops / (ms2 * 1e-3) / MFMA_BF16_DENSE_PEAK, 4),
          "speedup": round(ms2 / ms1, 3)}


def time_workload(dta, w, torch, warm_s=0.3, timed_s=0.2):
  """Prologue and attention times of one workload (HIP events), in steady
  state: each op first runs back to back for about ``warm_s`` seconds (the
  part ramps its clock over the first milliseconds of a burst: I1's first
  launches after an idle gap run ~10 % slower), then ``reps`` launches
  covering about ``timed_s`` seconds are timed."""
  from diffusers_tpu_amd.workloads import HBM_PEAK, MFMA_BF16_DENSE_PEAK
  x = w.inputs(device="cuda")
  v = x["v"].to(torch.bfloat16).contiguous()
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  kv_len = w.kv_len if w.padded else None
  qo = torch.empty((w.B, w.H, w.S, w.D), device="cuda", dtype=torch.bfloat16)
  ko = torch.empty_like(qo)
  out = torch.empty_like(qo)
  pro = lambda: dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps,
                                 rope=rope, q_head_scale=x["hs"],
                                 valid_len=kv_len, out=(qo, ko))
  ws = dta.splash.AttentionWorkspace()
  att = lambda: dta.attention(qo, ko, v, kv_len=kv_len, out=out, workspace=ws)
  res = {}
  for name, fn in (("prologue", pro), ("attention", att)):
    res[name + "_ms"], res[name + "_reps"] = _steady(fn, torch, warm_s,
                                                     timed_s)
  res["attention_tflops"] = round(w.attn_flops() / res["attention_ms"] / 1e9, 1)
  res["attention_pct_bf16_peak"] = round(
      100 * w.attn_flops() / (res["attention_ms"] * 1e-3) / MFMA_BF16_DENSE_PEAK, 2)
  res["prologue_GBs"] = round(w.prologue_bytes() / res["prologue_ms"] / 1e6, 1)
  res["prologue_pct_hbm_peak"] = round(
      100 * w.prologue_bytes() / (res["prologue_ms"] * 1e-3) / HBM_PEAK, 2)
  res["shape"] = f"B{w.B} H{w.H} S{w.S} D{w.D} kv_len {w.kv_len}"
  res["attention_frac"] = round(res["attention_pct_bf16_peak"] / 100, 4)
  return res


def gemm_ceiling(torch, n=8192, seconds=1.5):
  """Same-run clock-limited MFMA ceiling: a bf16 n^3 torch.matmul
  (hipBLASLt) on seeded N(0,1) operands, timed after a warm-up long enough
  for the part to settle at its power limit (MFMA throughput on this part
  depends on the operand values, so the ceiling is measured on random data
  like the attention operands)."""
  from diffusers_tpu_amd.workloads import MFMA_BF16_DENSE_PEAK
  g = torch.Generator(device="cuda").manual_seed(0)
  a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
  b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
  c = torch.empty_like(a)
  one = _time(lambda: torch.matmul(a, b, out=c), torch, 3)
  reps = max(10, int(seconds * 1e3 / one))
  _time(lambda: torch.matmul(a, b, out=c), torch, reps // 2)  # settle
  ms = _time(lambda: torch.matmul(a, b, out=c), torch, reps)
  tf = 2.0 * n ** 3 / (ms * 1e-3)
  return {"op": f"torch.matmul bf16 {n}^3 (hipBLASLt), N(0,1) operands",
          "ms": round(ms, 4), "TFLOPs": round(tf / 1e12, 1),
          "frac": round(tf / MFMA_BF16_DENSE_PEAK, 4), "reps": reps}


def zero_operand_ceilings(dta, w, torch, kv_len, n=8192, seconds=1.0):
  """The attention launch and the vendor GEMM on all-zero operands, in the
  same run: the instruction streams do not depend on the values, but zero
  operands toggle almost nothing, so the part is not held at its power
  limit and runs near its nominal clock.  Their ratio is the kernel's
  efficiency against the GEMM with power taken out of the comparison (the
  attention result on zeros is the mean of zero values; not a parity
  case)."""
  from diffusers_tpu_amd.workloads import MFMA_BF16_DENSE_PEAK
  shape = (w.B, w.H, w.S, w.D)
  z = torch.zeros(shape, device="cuda", dtype=torch.bfloat16)
  out = torch.empty_like(z)
  ms_att = _time(lambda: dta.splash._launch(z, z, z, None, kv_len, out=out),
                 torch, 3)
  del z, out
  a = torch.zeros(n, n, device="cuda", dtype=torch.bfloat16)
  c = torch.empty_like(a)
  one = _time(lambda: torch.matmul(a, a, out=c), torch, 3)
  reps = max(10, int(seconds * 1e3 / one))
  ms_g = _time(lambda: torch.matmul(a, a, out=c), torch, reps)
  att = w.attn_flops() / (ms_att * 1e-3)
  gemm = 2.0 * n ** 3 / (ms_g * 1e-3)
  return {"attention_ms": round(ms_att, 3),
          "attention_TFLOPs": round(att / 1e12, 1),
          "attention_frac": round(att / MFMA_BF16_DENSE_PEAK, 4),
          "gemm_TFLOPs": round(gemm / 1e12, 1),
          "gemm_frac": round(gemm / MFMA_BF16_DENSE_PEAK, 4),
          "attention_frac_of_gemm": round(att / gemm, 4),
          "note": "all-zero operands (not power-limited); diagnostic only"}


def hbm_ceiling(torch, nbytes, reps=20):
  """Same-run practical HBM ceiling: the best of the calibration copy
  kernels (csrc/calib/hbm_copy.hip: 16-byte non-temporal loads and
  stores, several grid shapes and loads in flight) moving nbytes/2 bytes,
  i.e. nbytes of read + write traffic, the prologue's byte count."""
  import ctypes
  from diffusers_tpu_amd import _build
  from diffusers_tpu_amd.workloads import HBM_PEAK
  lib = ctypes.CDLL(str(_build.CALIB_PATH))
  lib.dt_calib_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                ctypes.c_size_t, ctypes.c_int,
                                ctypes.c_void_p]
  half = int(nbytes // 2) // 16 * 16
  src = torch.randint(0, 255, (half,), device="cuda", dtype=torch.uint8)
  dst = torch.empty_like(src)
  stream = torch.cuda.current_stream().cuda_stream
  best = None
  for var in range(lib.dt_calib_copy_variants()):
    def run():
      if lib.dt_calib_copy(src.data_ptr(), dst.data_ptr(), half, var, stream):
        raise RuntimeError("dt_calib_copy failed")
    ms = _time(run, torch, reps)
    if best is None or ms < best[1]:
      best = (var, ms)
  if not torch.equal(src[:4096], dst[:4096]):
    raise RuntimeError("calibration copy produced wrong bytes")
  gbs = 2 * half / (best[1] * 1e-3) / 1e9
  return {"kernel": "calib copy (csrc/calib/hbm_copy.hip)",
          "bytes_read_plus_write": 2 * half, "best_variant": best[0],
          "ms": round(best[1], 4), "GBs": round(gbs, 1),
          "frac": round(gbs * 1e9 / HBM_PEAK, 4)}


def pattern_ceiling(torch, q, k, reps=20):
  """Same-run ceiling for the prologue's access pattern: the best of the
  calibration copies that read q and k [B, S, H, 128] bf16 and write them
  as [B, H, S, 128] (csrc/calib/hbm_copy.hip, dt_calib_bshd_copy: the
  prologue's own lane mapping and three head-major mappings), the same
  bytes the prologue moves, without its arithmetic."""
  import ctypes
  from diffusers_tpu_amd import _build
  from diffusers_tpu_amd.workloads import HBM_PEAK
  lib = ctypes.CDLL(str(_build.CALIB_PATH))
  lib.dt_calib_bshd_copy.argtypes = [ctypes.c_void_p] * 4 + \
      [ctypes.c_int] * 4 + [ctypes.c_void_p]
  b, s, h, d = q.shape
  if d != 128 or q.dtype != torch.bfloat16 or not q.is_contiguous() or \
     not k.is_contiguous():
    return None
  qo = torch.empty((b, h, s, d), device=q.device, dtype=q.dtype)
  ko = torch.empty_like(qo)
  stream = torch.cuda.current_stream().cuda_stream
  per = {}
  best = None
  for var in range(lib.dt_calib_bshd_copy_variants()):
    def run():
      if lib.dt_calib_bshd_copy(q.data_ptr(), k.data_ptr(), qo.data_ptr(),
                                ko.data_ptr(), b, s, h, var, stream):
        raise RuntimeError("dt_calib_bshd_copy failed")
    ms = _time(run, torch, reps)
    if not (torch.equal(qo[:, :, :64], q[:, :64].transpose(1, 2)) and
            torch.equal(ko[:, :, -64:], k[:, -64:].transpose(1, 2))):
      raise RuntimeError("pattern copy produced wrong bytes")
    per[var] = round(ms, 4)
    if best is None or ms < best[1]:
      best = (var, ms)
  nbytes = 4 * q.numel() * q.element_size()
  gbs = nbytes / (best[1] * 1e-3) / 1e9
  return {"kernel": "calib BSHD->BHSD copy (csrc/calib/hbm_copy.hip)",
          "bytes_read_plus_write": nbytes, "best_variant": best[0],
          "variant_ms": per, "ms": round(best[1], 4), "GBs": round(gbs, 1),
          "frac": round(gbs * 1e9 / HBM_PEAK, 4),
          "note": "variant 0 is the prologue's own lane mapping"}


def _time(fn, torch, reps):
  fn()
  torch.cuda.synchronize()
  e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
  e0.record()
  for _ in range(reps):
    fn()
  e1.record()
  torch.cuda.synchronize()
  return e0.elapsed_time(e1) / reps


class _PowerSampler:
  """Samples socket power, the mean gfx clock and the hotspot temperature
  with ``amd-smi metric -p -c -t --json`` (a read-only query, run as a
  child process) every ~0.4 s on
  a background thread; ``summary(t0, t1)`` averages the samples taken
  inside [t0, t1].  Without amd-smi it records nothing."""

  def __init__(self):
    import shutil
    import threading
    self.samples = []
    self.exe = shutil.which("amd-smi")
    self._stop = threading.Event()
    self._thread = threading.Thread(target=self._run, daemon=True)
    if self.exe:
      self._thread.start()

  def _run(self):
    import subprocess
    import time
    while not self._stop.is_set():
      t = time.time()
      try:
        r = subprocess.run([self.exe, "metric", "-p", "-c", "-t", "--json"],
                           capture_output=True, text=True, timeout=5)
        d = json.loads(r.stdout)
        g = d["gpu_data"][0] if isinstance(d, dict) else d[0]
        clk = [c["clk"]["value"] for k, c in g["clock"].items()
               if k.startswith("gfx_")]
        try:
          hot = float(g["temperature"]["hotspot"]["value"])
        except (KeyError, TypeError, ValueError):
          hot = float("nan")
        self.samples.append((t, float(g["power"]["socket_power"]["value"]),
                             sum(clk) / len(clk), hot))
      except Exception:  # a missing field or a failed query: skip the sample
        pass
      self._stop.wait(0.4)

  def stop(self):
    self._stop.set()
    if self.exe:
      self._thread.join(timeout=10)

  def summary(self, t0, t1):
    sel = [s for s in self.samples if t0 + 0.8 < s[0] < t1]
    if not sel:
      return None
    return {"samples": len(sel),
            "socket_power_W": round(sum(s[1] for s in sel) / len(sel), 1),
            "socket_power_max_W": max(s[1] for s in sel),
            "gfx_clock_MHz": round(sum(s[2] for s in sel) / len(sel), 1),
            "hotspot_C": round(sum(s[3] for s in sel) / len(sel), 1),
            "hotspot_max_C": max(s[3] for s in sel)}


def power_study(dta, w, torch, reps=16):
  """Attention and a vendor GEMM on random vs all-zero operands, with the
  socket power and gfx clock sampled during each (amd-smi).

  The instruction stream of the attention kernel does not depend on the
  values (the rare softmax re-base aside), so a time difference between the
  two inputs is the clock the part sustains under each operand toggle rate.
  """
  import time
  sampler = _PowerSampler()
  def timed(fn, n):
    fn()
    torch.cuda.synchronize()
    t0 = time.time()
    ms = _time(fn, torch, n)
    return ms, sampler.summary(t0, time.time())
  x = w.inputs(device="cuda")
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  kv_len = w.kv_len if w.padded else None
  qo, ko = dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps,
                            rope=rope, q_head_scale=x["hs"], valid_len=kv_len)
  v = x["v"].to(torch.bfloat16).contiguous()
  del x
  out = torch.empty_like(qo)
  res = {"workload": w.name, "attn_flops": w.attn_flops()}
  for name, (q, k, vv) in (("real", (qo, ko, v)),
                           ("zeros", (torch.zeros_like(qo),) * 3)):
    ms, pw = timed(lambda: dta.splash._launch(q, k, vv, None, kv_len,
                                              out=out), reps)
    res[f"attention_{name}"] = {"ms": round(ms, 3),
                                "TFLOPs": round(w.attn_flops() / ms / 1e9, 1),
                                "power": pw}
  del qo, ko, v, out
  n = 8192
  g = torch.Generator(device="cuda").manual_seed(0)
  a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
  b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
  for name, (x1, x2) in (("randn", (a, b)),
                         ("zeros", (torch.zeros_like(a), torch.zeros_like(b)))):
    ms, pw = timed(lambda: x1 @ x2, 5000)
    res[f"gemm_8192_bf16_{name}"] = {"ms": round(ms, 3),
                                     "TFLOPs": round(2 * n**3 / ms / 1e9, 1),
                                     "power": pw}
  sampler.stop()
  return res


def extras(dta, w, torch, qo, ko, v, out, kv_len, flops, packed):
  """Timings of the optional paths on the step's own tensors."""
  from diffusers_tpu_amd.workloads import HBM_PEAK
  # fixed-m path (kernels/splash.py:170-248): the bound's row-norm
  # reductions (HBM-bound, one read of q and one of k) as
  # attention(use_fixed_m=True) runs them (fixed_m_prepare: one grid over
  # q and k, then the operand), and the attention launch with the operand;
  # outside the timed step, which is the reference's default online path
  from diffusers_tpu_amd.kernels import fixed_m_bound as fmb
  mk = {}
  def bound():
    mk["v"] = fmb.fixed_m_prepare(qo, ko, None, smooth=False)[1]
  ms_bound = _time(bound, torch, 5)
  ms_fixed = _time(lambda: dta.splash._launch(qo, ko, v, None, kv_len, out=out,
                                              mk=mk["v"], packed_v=packed),
                   torch, 2)
  nb = 2 * qo.numel() * qo.element_size()
  fixed = {"row_norm_ms": round(ms_bound, 4),
           "row_norm_GBs": round(nb / ms_bound / 1e6, 1),
           "row_norm_frac_hbm": round(nb / (ms_bound * 1e-3) / HBM_PEAK, 4),
           "eligible_heads": int(mk["v"][1].sum().item()),
           "attention_ms": round(ms_fixed, 3),
           "attention_TFLOPs": round(flops / ms_fixed / 1e9, 1)}

  # qk_fp8 path (kernels/splash.py:420-424): the E4M3 key cast (HBM-bound)
  # and the attention launch with E4M3 q/k in the QK product
  from diffusers_tpu_amd.kernels.fp8_cast import quantize_saturating
  k8 = quantize_saturating(ko)
  ms_cast = _time(lambda: quantize_saturating(ko, out=k8), torch, 5)
  def att8():
    dta.splash._call_ex(qo, k8, 1, v, packed, out, False, w.H, w.S,
                        1.0 / w.D ** 0.5, kv_len or w.S, None)
  ms_att8 = _time(att8, torch, 2)
  cast_bytes = 3 * ko.numel()
  qk8 = {"cast_ms": round(ms_cast, 4),
         "cast_GBs": round(cast_bytes / ms_cast / 1e6, 1),
         "cast_frac_hbm": round(cast_bytes / (ms_cast * 1e-3) / HBM_PEAK, 4),
         "attention_ms": round(ms_att8, 3),
         "attention_TFLOPs": round(flops / ms_att8 / 1e9, 1),
         "note": "QK^T on E4M3 MFMA, PV bf16; TFLOP/s counts both products"}
  del k8

  # block-sparse temporal window (kernels/sparse_splash.py, the H3 table of
  # models/minimax_h3/h3_tpu.py:213-224): V7 has 87 latent frames of 48x84
  # rows; each video row keeps the key blocks within 8 frames of it
  from diffusers_tpu_amd.kernels import sparse_splash
  rpf = w.grid[1] * w.grid[2] if len(w.grid) == 3 else w.S
  table = sparse_splash.temporal_window_table(w.S, 0, rpf, 8, 2048, 2048)
  tt = sparse_splash.build_tile_table(table, sq=w.S, skv=w.S, heads=w.H,
                                      block_q=2048, block_kv=2048,
                                      kv_len=kv_len, device=qo.device)
  ms_sp = _time(lambda: sparse_splash.attention(
      qo, ko, v, scale=None, block_q=2048, block_kv=2048, kv_table=tt,
      kv_len=kv_len), torch, 2)
  sp_flops = flops * tt.kept_tiles / tt.full_tiles
  sparse = {"window_frames": 8, "rows_per_frame": rpf,
            "kept_tile_frac": round(tt.kept_tiles / tt.full_tiles, 4),
            "attention_ms": round(ms_sp, 3),
            "attention_TFLOPs_on_kept_tiles": round(sp_flops / ms_sp / 1e9, 1)}
  del tt

  return fixed, qk8, sparse


def prologue_table(dta, w, torch, x, qo, ko, kv_len):
  """The prologue with cos/sin read from per-token tables (the form H3's
  apply_rope and MOSS's _rotate take) instead of computed from positions:
  the same rotation as the timed step, plus the table reads."""
  freqs = []
  for a, dim in enumerate(w.axis_dims):
    i = torch.arange(dim // 2, dtype=torch.float64, device=qo.device)
    freqs.append(x["pos"][:, a:a + 1].double() * w.theta ** (-2.0 * i / dim))
  ang = torch.cat(freqs, -1)
  tab = dta.RopeTable(w.mode, torch.cos(ang).float(), torch.sin(ang).float())
  run = lambda: dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps,
                                 rope=tab, q_head_scale=x["hs"],
                                 valid_len=kv_len, out=(qo, ko))
  from diffusers_tpu_amd.workloads import HBM_PEAK
  ms = _time(run, torch, 20)
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  ms_pos = _time(lambda: dta.qk_norm_rope(
      x["q"], x["k"], x["wq"], x["wk"], eps=w.eps, rope=rope,
      q_head_scale=x["hs"], valid_len=kv_len, out=(qo, ko)), torch, 20)
  nb = w.prologue_bytes() + 2 * tab.cos.numel() * 4
  return {"kernel": "qk_norm_rope_kernel<D, RC, true>", "ms": round(ms, 4),
          "positions_ms": round(ms_pos, 4), "bytes": nb,
          "GBs": round(nb / ms / 1e6, 1),
          "frac_hbm": round(nb / (ms * 1e-3) / HBM_PEAK, 4)}


def main():
  ap = argparse.ArgumentParser()
  ap.add_argument("--gpus", type=int, default=1)
  ap.add_argument("--steps", type=int, default=10)
  ap.add_argument("--warmup", type=int, default=2)
  ap.add_argument("--workload", default="V7")
  ap.add_argument("--no-cpu-baseline", action="store_true")
  ap.add_argument("--no-workloads", action="store_true",
                  help="skip the per-workload prologue/attention timings of "
                       "the other BASELINE configs (P, I1, I2, V4) under "
                       "'workloads'")
  ap.add_argument("--no-ceilings", action="store_true",
                  help="skip the same-run GEMM and copy ceilings")
  ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                  help="only run a device-to-device copy of BYTES (the known-"
                       "size reference for HBM traffic counters) and exit")
  ap.add_argument("--no-extras", action="store_true",
                  help="skip the fixed-m, qk_fp8 and block-sparse timings that "
                       "follow the timed steps (e.g. under a kernel-trace "
                       "profiler, so its per-kernel averages cover the step)")
  ap.add_argument("--power-study", action="store_true",
                  help="only time the attention launch of the workload on its "
                       "real inputs and on all-zero inputs, and a bf16 8192^3 "
                       "torch.matmul (hipBLASLt) on N(0,1) and on zeros, then "
                       "exit: MFMA throughput on this part depends on the data")
  args = ap.parse_args()
  if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
    print("bench.py measures one GPU only: the attention path is benchmarked "
          "on one GPU's head shard (V7 = 5 of 40 heads); multi-GPU runs are "
          "not part of this build.", file=sys.stderr)
    sys.exit(2)

  import torch
  if args.copy_calibration:
    n = int(args.copy_calibration)
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    e0.record()
    dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    print(json.dumps({"copy_bytes": n, "ms": round(ms, 4),
                      "GBs_read_plus_write": round(2 * n / ms / 1e6, 1)}))
    return

  import diffusers_tpu_amd as dta
  from diffusers_tpu_amd.workloads import (HBM_PEAK, MFMA_BF16_DENSE_PEAK,
                                           WORKLOADS)
  if args.power_study:
    print(json.dumps(power_study(dta, WORKLOADS[args.workload], torch)),
          flush=True)
    return

  w = WORKLOADS[args.workload]
  dev = torch.device("cuda:0")
  x = w.inputs(device=dev)
  v = x["v"].to(torch.bfloat16).contiguous()
  rope = dta.RopeSpec(w.mode, x["pos"], w.axis_dims, w.theta)
  kv_len = w.kv_len if w.padded else None
  qo = torch.empty((w.B, w.H, w.S, w.D), device=dev, dtype=torch.bfloat16)
  ko = torch.empty_like(qo)
  out = torch.empty_like(qo)
  stream = torch.cuda.current_stream(dev)

  # the public entry point with a caller-owned workspace (packed-V buffer
  # and split workspace allocated once, on the first call)
  ws = dta.splash.AttentionWorkspace(dev)
  use_packed = (w.D == 128 and
                (kv_len or w.S) >= dta.splash.PACKED_V_MIN_KEYS)
  ev = []  # (prologue start, prologue end, attention end)

  def step(record):
    e0 = e1 = e2 = None
    if record:
      e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
      e0.record(stream)
    dta.qk_norm_rope(x["q"], x["k"], x["wq"], x["wk"], eps=w.eps, rope=rope,
                     q_head_scale=x["hs"], valid_len=kv_len, out=(qo, ko))
    if record:
      e1.record(stream)
    dta.attention(qo, ko, v, kv_len=kv_len, out=out, workspace=ws)
    if record:
      e2.record(stream)
      ev.append((e0, e1, e2))

  for _ in range(args.warmup):
    step(False)
  torch.cuda.synchronize()
  t_start = torch.cuda.Event(enable_timing=True)
  t_end = torch.cuda.Event(enable_timing=True)
  t_start.record(stream)
  for _ in range(args.steps):
    step(True)
  t_end.record(stream)
  torch.cuda.synchronize()
  ms_step = t_start.elapsed_time(t_end) / args.steps
  ms_pro = sum(a.elapsed_time(b) for a, b, _ in ev) / len(ev)
  ms_att = sum(b.elapsed_time(c) for _, b, c in ev) / len(ev)
  pack_bytes = 2 * v.numel() * v.element_size()  # read + write of V
  ms_pack = None
  if use_packed:  # the attention call's V pass, timed on its own
    vt = ws.packed_v(dta.splash.packed_v_numel(w.B, w.H, kv_len or w.S))
    ms_pack = _time(lambda: dta.splash.pack_v(v, kv_len, out=vt), torch, 10)
  vt = dta.splash.pack_v(v, kv_len)[0] if use_packed else None

  flops = w.attn_flops()
  tflops_step = flops / (ms_step * 1e-3) / 1e12
  att_tflops = flops / (ms_att * 1e-3) / 1e12
  peak_t = MFMA_BF16_DENSE_PEAK / 1e12
  # The prologue's launch duration: 20 back-to-back launches of the step's
  # own call between one pair of events.  A single ~0.3 ms launch bracketed
  # by its own events (ms_pro) carries the events' overhead, about 20-25 us
  # here; the kernel trace's in-step per-launch average agrees with this
  # figure instead (profiles/V7_kernel_trace.md).
  pro_call = lambda: dta.qk_norm_rope(
      x["q"], x["k"], x["wq"], x["wk"], eps=w.eps, rope=rope,
      q_head_scale=x["hs"], valid_len=kv_len, out=(qo, ko))
  ms_pro_launch = _time(pro_call, torch, 20)
  pro_gbs = w.prologue_bytes() / (ms_pro_launch * 1e-3) / 1e9

  fixed = qk8 = sparse = table = None
  if not args.no_extras:
    packed = dta.splash.pack_v(v, kv_len, out=vt) if use_packed else None
    fixed, qk8, sparse = extras(dta, w, torch, qo, ko, v, out, kv_len, flops,
                                packed)
    table = prologue_table(dta, w, torch, x, qo, ko, kv_len)

  gemm = hbm = zeros = pattern = None
  if not args.no_ceilings:
    gemm = gemm_ceiling(torch)
    hbm = hbm_ceiling(torch, w.prologue_bytes())
    pattern = pattern_ceiling(torch, x["q"], x["k"])
    zeros = zero_operand_ceilings(dta, w, torch, kv_len)

  workloads = None
  if not args.no_workloads:
    workloads = {n: time_workload(dta, wl, torch)
                 for n, wl in WORKLOADS.items() if n != w.name}
    workloads["I1_cfg_pair"] = cfg_pair(dta, torch)

  cpu = None
  if not args.no_cpu_baseline:
    cpu = cpu_baseline(w, (qo.float().cpu(), ko.float().cpu(),
                           v.float().cpu()))

  roof = {"kernel": "flash_attn_kernel", "bound": "mfma",
          "achieved": round(att_tflops, 2), "peak": peak_t,
          "unit": "TFLOP/s", "frac": round(att_tflops / peak_t, 4),
          "ms": round(ms_att, 3),
          "timed": "the attention() call in each timed step (HIP events on "
                   "its stream): the flash kernel plus the packed-V pass "
                   "and the split merge (about 0.1 % of the call)",
          "traffic": _traffic("flash_fwd", w.name)}
  pro = {"kernel": "qk_norm_rope_kernel", "bound": "hbm",
         "achieved": round(pro_gbs, 1), "peak": HBM_PEAK / 1e9,
         "unit": "GB/s", "frac": round(pro_gbs * 1e9 / HBM_PEAK, 4),
         "ms": round(ms_pro_launch, 4),
         "timed": "20 back-to-back launches of the step's prologue call "
                  "between one pair of HIP events, right after the timed "
                  "steps",
         "in_step_event_ms": round(ms_pro, 4),
         "algorithmic_bytes": w.prologue_bytes(),
         "traffic": _traffic("qk_norm_rope", w.name)}
  if gemm is not None:
    roof["frac_of_gemm_ceiling"] = round(att_tflops / gemm["TFLOPs"], 4)
  if hbm is not None:
    pro["frac_of_copy_ceiling"] = round(pro_gbs / hbm["GBs"], 4)
  if pattern is not None:
    pro["frac_of_pattern_ceiling"] = round(pro_gbs / pattern["GBs"], 4)
  line = {
      "metric": METRIC,
      "value": round(tflops_step, 2),
      "unit": "TFLOP/s",
      "n_gpus": 1,
      "steps": args.steps,
      "warmup": args.warmup,
      "ms_per_step": round(ms_step, 3),
      "higher_is_better": True,
      "scaling": "weak",
      "vs_baseline": None,
      "dtype": "bf16",
      "data": "synthetic (seeded N(0,1) q/k/v, RMSNorm weights N(1,0.02))",
      "config": {"workload": f"{w.name}: {w.desc}",
                 "B": w.B, "H": w.H, "S": w.S, "D": w.D,
                 "kv_len": w.kv_len, "rope": f"{w.mode} {w.axis_dims}",
                 "attn_flops": flops},
      "ms_per_layer": round(ms_step, 3),
      "pct_bf16_peak": round(100 * tflops_step / peak_t, 2),
      "roofline": roof,
      "prologue": pro,
      "pack_v": ({"kernel": "v_pack_kernel", "bound": "hbm",
                  "ms": round(ms_pack, 4),
                  "GBs": round(pack_bytes / ms_pack / 1e6, 1),
                  "note": "V into the tile-major packed layout the attention "
                          "kernel streams (read + write of V)"}
                 if use_packed else None),
      "fixed_m": fixed,
      "qk_fp8": qk8,
      "sparse_window": sparse,
      "prologue_table": table,
      "gemm_ceiling": gemm,
      "hbm_ceiling": hbm,
      "pattern_ceiling": pattern,
      "zero_operands": zeros,
      "cpu_baseline": cpu,
  }
  if workloads is not None:
    line["workloads"] = workloads
  print(json.dumps(line), flush=True)


if __name__ == "__main__":
  main()
