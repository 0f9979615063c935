"""FP8 linear training caller of the gfx950 fp8 GEMM.

This package provides only ``train.fp8``. Its search path is extended over every
``train`` directory on ``sys.path`` (pkgutil.extend_path), so a reference checkout
placed after this directory still supplies the model, config, training loop and
parallel modules, which then bind this ``train.fp8``.
"""

import pkgutil

__path__ = pkgutil.extend_path(__path__, __name__)
