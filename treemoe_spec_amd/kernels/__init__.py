"""HIP-backed op1 / op4 operators (same names as treemoe/kernels)."""
