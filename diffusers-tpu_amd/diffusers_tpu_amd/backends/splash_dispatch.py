"""Route diffusers' attention dispatch to the gfx950 kernel.

Mirror of ``diffusers_tpu/backends/ours_splash_tt.py:45-231`` for torch on
ROCm.  Two pieces:

* a registered torch op, ``dt::splash_attention``, with a shape-only fake so
  Dynamo / ``torch.compile`` trace through it without running the kernel
  (the reference registers a ``pallas::h3_splash_*`` op with the same kind
  of fake, :45-77);
* ``make_dispatch(original)``, a drop-in for
  ``diffusers.models.attention_dispatch.dispatch_attention_fn`` that sends
  the mask-free, non-causal, dropout-free calls on long sequences to that
  op and everything else to ``original`` (:92-157).  Layout: diffusers
  passes ``(B, S, H, D)``; the op takes ``(B, H, S, D)``; the result is
  ``(B, S, H, D)`` for every caller, also those that pass
  ``_already_bhsd=True`` (:149-152).  With fixed-m the keys are k-smoothed
  first (``k - mean_S(k)``), which fixed-m's no-flush gate presumes
  (:136-137);
* ``make_processor_call(orig_call, dispatch)``, the BHSD-first attention
  processor (:165-231): projections, then QK-RMSNorm and RoPE as one
  ``qk_norm_rope`` pass that reads the ``(B, S, H, D)`` projection views
  and the processor's ``(cos, sin)`` tables in place and writes
  ``(B, H, S, D)``, then the dispatch, then the output projection.

``install()`` patches diffusers in place when it is importable.
"""
from __future__ import annotations

import os

import torch

# kernels/splash block sizes are TPU tiling knobs; kept for the op's name
# parity only.  Shorter sequences go to the original dispatch (:37-39).
MIN_SEQ = int(os.environ.get("DT_OURS_MIN_SEQ", "2048"))
QK_FP8 = os.environ.get("DT_OURS_QK_FP8") == "1"
# Sparse op and the sequence length it serves, or None / 0 for dense (:43-44).
SPARSE_OP = None
SPARSE_SEQ = 0


@torch.library.custom_op("dt::splash_attention", mutates_args=())
def splash_attention(query: torch.Tensor, key: torch.Tensor,
                     value: torch.Tensor, use_fixed_m: bool = False,
                     qk_fp8: bool = False,
                     smooth_k: bool = False) -> torch.Tensor:
  """``kernels.splash.attention`` with the default scale, ``(B,H,S,D)``.

  ``smooth_k``: subtract the keys' mean first (``k_smoothing.smooth_keys``);
  with ``use_fixed_m`` the bound then takes the smoothed keys' norms from
  that pass instead of a second read of k."""
  from ..kernels import fixed_m_bound, k_smoothing, splash
  mk = None
  if smooth_k:
    if use_fixed_m:  # smoothing, both norms and the operand: three launches
      key, mk = fixed_m_bound.fixed_m_prepare(query, key, smooth=True)
    else:
      key = k_smoothing.smooth_keys(key)
  return splash._attention(query, key, value, None, use_fixed_m, qk_fp8,
                           None, mk=mk)


@splash_attention.register_fake
def _splash_attention_fake(query, key, value, use_fixed_m=False,
                           qk_fp8=False, smooth_k=False):
  # output = query's shape and dtype (ours_splash_tt.py:68-75)
  return torch.empty_like(query, memory_format=torch.contiguous_format)


@torch.library.custom_op("dt::smooth_keys", mutates_args=())
def smooth_keys_op(key: torch.Tensor) -> torch.Tensor:
  """``key - mean_S(key)`` on ``(B,H,S,D)`` (k_smoothing.smooth_keys)."""
  from ..kernels import k_smoothing
  return k_smoothing.smooth_keys(key)


@smooth_keys_op.register_fake
def _smooth_keys_fake(key):
  return torch.empty_like(key, memory_format=torch.contiguous_format)


class KernelDispatch:
  """diffusers' ``dispatch_attention_fn`` with the eligible calls served by
  the gfx950 kernel (the contract of ours_splash_tt.py:92-157).

  A call is eligible when it has no mask, no dropout, is not causal and both
  sequences reach ``min_seq``; every other call goes to ``original``
  unchanged.  Layouts: diffusers passes ``(B, S, H, D)``, or
  ``(B, H, S, D)`` with ``_already_bhsd=True``; the kernel takes
  ``(B, H, S, D)``; the result is ``(B, S, H, D)`` for every caller.
  ``stats`` counts the two routes (``"n"`` kernel calls, ``"fallback"``),
  outside of ``torch.compile`` tracing.
  """

  def __init__(self, original, *, fixed_m=True, qk_fp8=QK_FP8,
               min_seq=MIN_SEQ, op=None, verbose=None):
    self.original = original
    self.fixed_m = fixed_m
    self.qk_fp8 = qk_fp8
    self.min_seq = min_seq
    self.op = op
    self.verbose = verbose
    self.stats = {"n": 0, "fallback": 0}

  def _refusal(self, query, key, attn_mask, dropout_p, is_causal, seq_ax):
    """Why the kernel cannot take this call, or None."""
    if attn_mask is not None:
      return f"mask {tuple(attn_mask.shape)}"
    if dropout_p:
      return f"dropout {dropout_p}"
    if is_causal:
      return "causal"
    if min(query.shape[seq_ax], key.shape[seq_ax]) < self.min_seq:
      return f"sequence {query.shape[seq_ax]}/{key.shape[seq_ax]} < " \
             f"{self.min_seq}"
    return None

  def _kernel(self, q, k, v):
    """Attention on (B, H, S, D) operands."""
    if SPARSE_OP is not None and q.shape[-2] == SPARSE_SEQ:
      if self.fixed_m:
        k = torch.ops.dt.smooth_keys(k)
      return SPARSE_OP(q, k, v)
    if self.op is not None:
      if self.fixed_m:
        k = k - k.mean(dim=-2, keepdim=True)
      return self.op(q, k, v)
    # k-smoothing runs inside the op, fused with the fixed-m bound
    return torch.ops.dt.splash_attention(q, k, v, self.fixed_m, self.qk_fp8,
                                         self.fixed_m)

  def __call__(self, query, key, value, attn_mask=None, dropout_p=0.0,
               is_causal=False, **kwargs):
    bhsd = kwargs.pop("_already_bhsd", False)
    to_other = lambda ts: [t.transpose(1, 2) for t in ts]
    count = not torch.compiler.is_compiling()
    why = self._refusal(query, key, attn_mask, dropout_p, is_causal,
                        -2 if bhsd else -3)
    if why is None:
      if count:
        self.stats["n"] += 1
      q, k, v = (query, key, value) if bhsd else to_other((query, key, value))
      return self._kernel(q, k, v).transpose(1, 2)
    if count:
      self.stats["fallback"] += 1
      if self.stats["fallback"] == 1 and self.verbose is not None:
        self.verbose(f"  [dt] first fallback ({why}): q={tuple(query.shape)}")
    if bhsd:
      query, key, value = to_other((query, key, value))
    return self.original(query, key, value, attn_mask=attn_mask,
                         dropout_p=dropout_p, is_causal=is_causal, **kwargs)


def make_dispatch(original, *, fixed_m: bool = True, qk_fp8: bool = QK_FP8,
                  min_seq: int = MIN_SEQ, op=None, verbose=None):
  """The replacement dispatch function (ours_splash_tt.py:92-157): a
  ``KernelDispatch`` over ``original`` (the fallback).  ``op``: the
  attention callable on ``(B, H, S, D)`` tensors, default
  ``dt::splash_attention``."""
  return KernelDispatch(original, fixed_m=fixed_m, qk_fp8=qk_fp8,
                        min_seq=min_seq, op=op, verbose=verbose)


class _HalvesCache:
  """Remembers, per (cos, sin) table pair, whether the second half of each
  repeats the first (``check_halves``, one host sync per new table): the
  fused prologue reads only the first half.

  An entry holds weak references to the two tensors and their version
  counters: it answers only for those same tensor objects, unmodified.  A
  table freed and reallocated at the same address is another object and is
  checked again, as is one updated in place.  While tracing
  (``torch.compile``) the values are not available, so the answer is
  ``False`` and the caller takes the stock processor: a table is never
  rotated by the fused kernel without its halves having been checked."""

  def __init__(self, size=64):
    self.size = size
    self.seen = {}

  def __call__(self, cos, sin):
    import weakref
    from ..kernels.qk_norm_rope import check_halves
    if torch.compiler.is_compiling():
      return False  # data-dependent checks cannot run while tracing
    key = (id(cos), id(sin))
    hit = self.seen.get(key)
    if hit is not None:
      wc, ws, vc, vs, ok = hit
      if wc() is cos and ws() is sin and vc == cos._version and \
         vs == sin._version:
        return ok
    ok = check_halves(cos, sin)
    if len(self.seen) >= self.size:
      self.seen.clear()
    self.seen[key] = (weakref.ref(cos), weakref.ref(sin), cos._version,
                      sin._version, ok)
    return ok


def _rms_operands(norm, d):
  """(weight, eps) of an RMSNorm module (diffusers' ``RMSNorm`` or
  ``torch.nn.RMSNorm``), or None when it is something else."""
  if not hasattr(norm, "eps") or not hasattr(norm, "weight"):
    return None
  if type(norm).__name__ not in ("RMSNorm", "FP32RMSNorm"):
    return None
  w = norm.weight
  if w is None:
    w = torch.ones(d)
  eps = norm.eps
  if eps is None:                      # torch.nn.RMSNorm default
    eps = torch.finfo(torch.float32).eps
  return w.detach(), float(eps)


# head dims the fused QK-RMSNorm + RoPE kernel is built for
PROLOGUE_HEAD_DIMS = (64, 128)


def make_processor_call(orig_call, dispatch, *, min_seq: int = MIN_SEQ):
  """The BHSD-first ``AttnProcessor.__call__`` (ours_splash_tt.py:165-231).

  ``orig_call(self, attn, hidden_states, rotary_emb, attention_mask)`` is
  the processor method it replaces and serves the calls the kernels do not
  (an attention mask, sequences shorter than ``min_seq``, norms that are
  not RMSNorm or whose epsilons differ, head dims other than 64 and 128,
  rotary tables whose halves differ).  ``rotary_emb`` is diffusers'
  ``(cos, sin)`` pair of ``(S, rotary)`` tables with repeated halves
  (rotate-half over the leading ``rotary`` channels, the rest pass
  through); each new table pair is checked once.  ``dispatch`` is the
  ``make_dispatch`` result; it returns ``(B, S, H, D)``.
  """
  from ..kernels.qk_norm_rope import RopeTable, qk_norm_rope
  halves_ok = _HalvesCache()

  def call(self, attn, hidden_states, rotary_emb=None, attention_mask=None):
    if attention_mask is not None or hidden_states.shape[-2] < min_seq:
      return orig_call(self, attn, hidden_states, rotary_emb, attention_mask)
    if getattr(attn, "fused_projections", False):
      query, key, value = attn.to_qkv(hidden_states).chunk(3, dim=-1)
    else:
      query = attn.to_q(hidden_states)
      key = attn.to_k(hidden_states)
      value = attn.to_v(hidden_states)
    # (B, S, H, D) views of the projections; the prologue reads them with
    # their strides, so a fused qkv output is not copied
    query, key, value = (t.unflatten(-1, (attn.heads, -1))
                         for t in (query, key, value))
    d = query.shape[-1]
    nq = _rms_operands(attn.norm_q, d)
    nk = _rms_operands(attn.norm_k, d)
    if (nq is None or nk is None or nq[1] != nk[1]
        or d not in PROLOGUE_HEAD_DIMS):
      return orig_call(self, attn, hidden_states, rotary_emb, attention_mask)
    rope = None
    if rotary_emb is not None:
      cos, sin = rotary_emb
      # the kernel reads the first half of each table; a table whose halves
      # differ rotates otherwise, so it goes to the original processor
      if not halves_ok(cos, sin):
        return orig_call(self, attn, hidden_states, rotary_emb,
                         attention_mask)
      rope = RopeTable.from_cos_sin(cos, sin)
    q, k = qk_norm_rope(query, key, nq[0], nk[0], eps=nq[1], rope=rope)
    out = dispatch(q, k, value.transpose(1, 2), attn_mask=None,
                   dropout_p=0.0, is_causal=False, _already_bhsd=True)
    out = out.flatten(2, 3).type_as(query)
    out = attn.to_out[0](out)
    return attn.to_out[1](out)

  return call


def install(verbose=print, fixed_m: bool = True) -> bool:
  """Patch diffusers' attention dispatch (ours_splash_tt.py:80-160).

  Returns False (and reports why) when diffusers is not importable.
  """
  try:
    from diffusers.models import attention_dispatch
  except ImportError as exc:
    verbose(f"  [dt] diffusers not importable ({exc}); nothing patched")
    return False
  dispatch = make_dispatch(attention_dispatch.dispatch_attention_fn,
                           fixed_m=fixed_m, verbose=verbose)
  attention_dispatch.dispatch_attention_fn = dispatch
  for mod in ("transformer_minimax_h3", "transformer_minimax_h3_image"):
    try:
      m = __import__(f"diffusers.models.transformers.{mod}", fromlist=["_"])
    except ImportError:
      continue
    if hasattr(m, "dispatch_attention_fn"):
      m.dispatch_attention_fn = dispatch
    # BHSD-first processor (ours_splash_tt.py:170-228); DT_BHSD_ROPE=0
    # keeps diffusers' own processor
    if os.environ.get("DT_BHSD_ROPE", "1") != "0":
      for cls in ("MiniMaxH3AttnProcessor", "MiniMaxH3ImageAttnProcessor"):
        proc = getattr(m, cls, None)
        if proc is not None:
          proc.__call__ = make_processor_call(proc.__call__, dispatch)
          verbose(f"  [dt] {cls}: fused norm + RoPE prologue")
  verbose("  [dt] attention routed to the gfx950 kernel")
  return True
