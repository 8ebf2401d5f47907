"""CPU oracle for the DiT attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy (float64) and plain torch-CPU (float32), the
arithmetic of the reference's attention path (shungcp/diffusers-tpu):

* ``attention``  — dense softmax attention with a runtime key-length mask,
  restating ``diffusers_tpu/kernels/splash.py:566-650`` (normalized output) and
  its XLA fallbacks ``models/moss_image/jax_dit.py:183-187`` /
  ``models/minimax_h3/jax_dit.py:393-399``; plus the residual ``(o, m, l)``
  form of ``kernels/splash.py:665-742``.
* ``norm_rope``  — QK-RMSNorm and RoPE (rotate-half and interleaved-pair
  conventions with per-axis channel splits), restating
  ``models/minimax_h3/jax_dit.py:184-195,251-262,603-617``,
  ``models/qwen_image_21/jax_dit.py:182-192,214-220`` and
  ``models/moss_image/jax_dit.py:126-142``.
* ``fixed_m``    — the host-side Cauchy-Schwarz bound
  ``kernels/fixed_m_bound.py:57-118`` and the key smoothing it presumes
  (``models/minimax_h3/jax_server.py:271-289``).
* ``fp8``        — the saturating E4M3 cast of ``kernels/fp8_cast.py:28-39``
  (qk_fp8).
* ``sparse``     — block-sparse attention semantics
  (``kernels/sparse_splash.py``) and the H3 temporal-window table
  (``models/minimax_h3/h3_tpu.py:213-224``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker.  The product path
(``diffusers_tpu_amd``) never imports it and has no CPU fallback.

Pinning (what fixes each function independently of its own formula) lives in
``tests/test_oracle.py``; every function here is pinned there.
"""
