"""Serving-side quantization for the gfx950 quantized-linear path."""
