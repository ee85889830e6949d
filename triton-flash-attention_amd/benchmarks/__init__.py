"""Benchmark harness for the gfx950 FlashAttention kernels."""
