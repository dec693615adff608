"""FP8 attention kernels (gfx950)."""
