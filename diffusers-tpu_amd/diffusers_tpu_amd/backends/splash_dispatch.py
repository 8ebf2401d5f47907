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
  passes ``(B, S, H, D)``; the op takes ``(B, H, S, D)``.  With fixed-m the
  keys are k-smoothed first (``k - mean_S(k)``), which fixed-m's no-flush
  gate presumes (:136-137).

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
                     qk_fp8: bool = False) -> torch.Tensor:
  """``kernels.splash.attention`` with the default scale, ``(B,H,S,D)``."""
  from ..kernels import splash
  return splash.attention(query, key, value, scale=None, block_q=0,
                          block_kv=0, block_kv_compute=0,
                          use_fixed_m=use_fixed_m, qk_fp8=qk_fp8)


@splash_attention.register_fake
def _splash_attention_fake(query, key, value, use_fixed_m=False,
                           qk_fp8=False):
  # output = query's shape and dtype (ours_splash_tt.py:68-75)
  return torch.empty_like(query, memory_format=torch.contiguous_format)


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
  kernel = op if op is not None else (
      lambda q, k, v: torch.ops.dt.splash_attention(q, k, v, fixed_m, qk_fp8))
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
    if fixed_m:
      key = key - key.mean(dim=-2, keepdim=True)
    if not tracing:
      state["n"] += 1
    if SPARSE_OP is not None and query.shape[-2] == SPARSE_SEQ:
      out = SPARSE_OP(query, key, value)
    else:
      out = kernel(query, key, value)
    return out if already_bhsd else out.transpose(1, 2)

  dispatch.stats = state
  return dispatch


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
  verbose("  [dt] attention routed to the gfx950 kernel")
  return True
