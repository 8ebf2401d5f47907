"""Integrations of the gfx950 attention kernels into torch model code."""
