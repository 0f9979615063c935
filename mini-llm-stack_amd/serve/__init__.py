"""Serving-side quantization for the gfx950 quantized-linear path.

This package provides only ``serve.quantize``. Its search path is extended over
every ``serve`` directory on ``sys.path`` (pkgutil.extend_path), so a reference
checkout placed after this directory still supplies the engine, KV cache,
speculative decoding and API modules, which then bind this ``serve.quantize``.
"""

import pkgutil

__path__ = pkgutil.extend_path(__path__, __name__)
