"""FP8 attention and FP8 block-scaled linear kernels (gfx950)."""
