"""MI355X (gfx950) drop-in for MetalNative's quantized-weight linear path.

Mirrors the reference's Python surface for this path
(python/metal_native/__init__.py:23-46 exposes ``_C``): ``_C.dequant_matmul``,
``_C.matmul``, ``_C.fast.swiglu``, ``_C.synchronize`` and
``_C.MetalNativeError``, on PyTorch-ROCm tensors.  The kernels are HIP code for
gfx950 in libmetal_native_amd.so; importing this package without the built
library raises ImportError (there is no CPU fallback).
"""

from __future__ import annotations

import types

from .ops import (MetalNativeError, dequant_matmul, dequantize, last_path, matmul, quantize,
                  set_option, swiglu, synchronize)

from . import nn, qformat  # noqa: E402  (layers, on-disk format and converters)
from .qcache import QuantWeightCache  # noqa: E402

fast = types.SimpleNamespace(swiglu=swiglu)

# reference-style `_C` namespace (bindings/bind_core.cpp:102)
_C = types.SimpleNamespace(
    dequant_matmul=dequant_matmul,
    matmul=matmul,
    fast=fast,
    synchronize=synchronize,
    MetalNativeError=MetalNativeError,
)

__all__ = ["MetalNativeError", "dequant_matmul", "dequantize", "quantize", "matmul", "swiglu",
           "fast", "synchronize", "set_option", "last_path", "_C", "nn", "qformat", "QuantWeightCache"]
