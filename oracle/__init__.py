"""CPU oracle for the gfx950 FlashAttention kernels (test infrastructure only)."""
