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


def make_dispatch(original, *, fixed_m: bool = True, qk_fp8: bool = QK_FP8,
                  min_seq: int = MIN_SEQ, op=None, verbose=None):
  """The replacement dispatch function (ours_splash_tt.py:92-157).

  ``original``: the function it replaces (the fallback).  ``op``: the
  attention callable on ``(B, H, S, D)`` tensors, default
  ``dt::splash_attention``.  Returns a function with diffusers'
  ``dispatch_attention_fn(query, key, value, attn_mask=None,
  dropout_p=0.0, is_causal=False, **kwargs)`` signature; ``stats`` on it
  counts kernel hits and fallbacks.
  """
  if op is not None:
    def kernel(q, k, v):
      if fixed_m:
        k = k - k.mean(dim=-2, keepdim=True)
      return op(q, k, v)
  else:
    # k-smoothing runs inside the op, fused with the fixed-m bound
    kernel = lambda q, k, v: torch.ops.dt.splash_attention(q, k, v, fixed_m,
                                                           qk_fp8, fixed_m)
  state = {"n": 0, "fallback": 0}

  def dispatch(query, key, value, attn_mask=None, dropout_p=0.0,
               is_causal=False, **kwargs):
    already_bhsd = kwargs.pop("_already_bhsd", False)
    seq_ax = -2 if already_bhsd else -3
    tracing = torch.compiler.is_compiling()
    if (attn_mask is not None or dropout_p or is_causal
        or query.shape[seq_ax] < min_seq or key.shape[seq_ax] < min_seq):
      if not tracing:
        state["fallback"] += 1
        if state["fallback"] == 1 and verbose is not None:
          verbose(f"  [dt] fallback: q={tuple(query.shape)} mask="
                  f"{None if attn_mask is None else tuple(attn_mask.shape)}"
                  f" causal={is_causal} dropout={dropout_p}")
      if already_bhsd:
        query, key, value = (t.transpose(1, 2) for t in (query, key, value))
      return original(query, key, value, attn_mask=attn_mask,
                      dropout_p=dropout_p, is_causal=is_causal, **kwargs)
    if not already_bhsd:
      query, key, value = (t.transpose(1, 2) for t in (query, key, value))
    if not tracing:
      state["n"] += 1
    if SPARSE_OP is not None and query.shape[-2] == SPARSE_SEQ:
      if fixed_m:
        key = torch.ops.dt.smooth_keys(key)
      out = SPARSE_OP(query, key, value)
    else:
      out = kernel(query, key, value)
    return out.transpose(1, 2)   # (B, S, H, D) for every caller

  dispatch.stats = state
  return dispatch


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
  not RMSNorm or whose epsilons differ, head dims other than 64 and 128).  ``rotary_emb`` is diffusers'
  ``(cos, sin)`` pair of ``(S, rotary)`` tables with repeated halves
  (rotate-half over the leading ``rotary`` channels, the rest pass
  through).  ``dispatch`` is the ``make_dispatch`` result; it returns
  ``(B, S, H, D)``.
  """
  from ..kernels.qk_norm_rope import RopeTable, qk_norm_rope

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
