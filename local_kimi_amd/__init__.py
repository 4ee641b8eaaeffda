"""MI355X-native W4A16 / MXFP4 quantized-matmul path of the local-kimi engine.

``local_kimi_amd.kernels`` registers the ops behind the reference's kernel
registry; ``local_kimi_amd.quant`` holds the packed INT4 codec. All compute
runs in the gfx950 HIP library ``liblkamd.so`` built from ``csrc/``.
"""

from . import _lib

__all__ = ["_lib"]
