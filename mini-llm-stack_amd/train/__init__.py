"""FP8 linear training caller of the gfx950 fp8 GEMM."""
