"""SDPA-shaped adapter over the gfx950 attention kernel.

Mirrors ``diffusers_tpu/kernels/mesh_attention.py::configure``
(:148-263), whose ``_sdpa`` closure (:218-261) is the callable the
reference's torch-side pipelines call as
``sdpa(query, key, value, attn_mask, dropout_p, is_causal, scale,
enable_gqa)`` on ``[B, H, S, D]`` tensors.  On one MI355X there is no mesh
to place the call on, so the adapter is only the dispatch to
``splash.attention``.

Differences from the reference, all explicit:

* The reference drops ``attn_mask``/``dropout_p``/``is_causal`` silently
  (:228); this adapter raises ``NotImplementedError`` for them rather than
  returning a result that ignores them.  Key padding is expressed with
  ``kv_len`` (``splash.attention``), as the reference's kernels do.
* k-smoothing (``key - mean_S(key)``, :234-237) exists in the reference to
  keep its fixed-m softmax in range (zero-mean keys give every row
  rowmax >= 0, which the fixed-m gate rests on); softmax is invariant to
  it.  The reference always applies it; here it follows ``use_fixed_m`` by
  default (the online softmax does not need it), and ``k_smoothing``
  forces it on or off.  Under ``kv_len`` the mean is over the real rows and
  the padded rows stay zero (models/minimax_h3/jax_server.py:278-281); it
  runs as ``k_smoothing.smooth_keys``, whose pass also yields the keys' half
  of the fixed-m bound.
"""
from __future__ import annotations

from . import fixed_m_bound
from . import k_smoothing as _ksm
from . import splash

KERNELS = ("custom_splash",)


def configure(kernel: str = "custom_splash", block_q=None, block_kv=None,
              block_kv_compute=None, use_fixed_m: bool = False,
              qk_fp8: bool = False, k_smoothing: bool | None = None):
  """Returns ``sdpa(query, key, value, attn_mask=None, dropout_p=0.0,
  is_causal=False, scale=None, enable_gqa=False)`` over ``[B, H, S, D]``.

  Raises:
    ValueError: if ``kernel`` names no kernel of this build (as
      mesh_attention.py:181-185).
  """
  smooth = use_fixed_m if k_smoothing is None else bool(k_smoothing)
  if kernel not in KERNELS:
    raise ValueError(f"attention {kernel!r} is not a kernel of this build; use"
                     f" one of {list(KERNELS)}")

  def sdpa(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
           scale=None, enable_gqa=False, kv_len=None):
    if attn_mask is not None or dropout_p or is_causal:
      raise NotImplementedError(
          "attn_mask / dropout / causal are not supported by the attention "
          "kernel; express key padding with kv_len")
    if query.shape[1] != key.shape[1] and not enable_gqa:
      raise ValueError("query and key head counts differ; pass enable_gqa=True")
    mk = None
    if smooth:
      # kv_len: an int or a device scalar (read by the kernels at run time)
      if use_fixed_m:
        key, mk = fixed_m_bound.fixed_m_prepare(query, key, scale,
                                                kv_len=kv_len, smooth=True)
      else:
        key = _ksm.smooth_keys(key, kv_len)
    return splash._attention(query, key, value, scale, use_fixed_m, qk_fp8,
                             kv_len, mk=mk)

  return sdpa
