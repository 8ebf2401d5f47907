"""Attention-path kernels (mirrors ``diffusers_tpu/kernels``)."""
