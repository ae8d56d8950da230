"""glypr_amd — MI355X (gfx950) HIP backend for glypr's Q8_0 hot path.

The product is libglypr_hip.so (C ABI in include/glypr_hip.h), built in-tree by
`python -m glypr_amd.build`.  `glypr_amd.ops` wraps it for torch tensors.
"""
from ._lib import (BF16_DEQUANT, INT8_EXACT, INT8_FMA, LIB_PATH, GlyprError, check, last_error, lib)

__all__ = ["BF16_DEQUANT", "INT8_EXACT", "INT8_FMA", "LIB_PATH", "GlyprError", "check",
           "last_error", "lib"]
