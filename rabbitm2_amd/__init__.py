"""MI355X (gfx950) MoE-layer path for the RABBIT2 engine.

The product is the C-ABI shared library librbt2_hip.so (header: include/rbt2_hip.h) built from
csrc/ by build.py; hip.py is a ctypes view of that ABI for Python hosts.
"""
from .hip import (DT_BF16, DT_F32, ORDER_AVX2, ORDER_SCALAR, Device, HipError, MoeLayer,  # noqa: F401
                  moe_layer_desc)
