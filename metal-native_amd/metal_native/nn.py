"""Linear layers on the library's kernels.

``Linear`` mirrors the reference's python/metal_native/nn/linear.py:9-55
(``y = x @ W^T + b`` through ``_C.matmul(x, W, False, True)``, Xavier-uniform
weights, zero bias) on fp16 GPU tensors: the M <= 8 rows run on the library's
vecmat kernel, other shapes on torch.matmul as in ``metal_native.matmul``.

``QuantizedLinear`` is the quantized counterpart the reference lacks: int4 /
int8 weights in the reference's storage format with the bias fused into the
GEMV/GEMM epilogue (``dequant_matmul(..., epilogue="bias")``).  The library
picks the kernel by the number of rows: the row-block GEMV for M <= 4, and
up to M = 16 where the activations fit in LDS; for int4 at M = 5..16 the
register-streamed GEMV where its plan takes the shape; the split-K GEMV for
short rows and what the others decline; the MFMA GEMM beyond M = 16.  Built from fp16 weights (``from_float``, quantized on the GPU by
``quantize``) or from a ``QuantizedWeight`` (a loaded or converted
checkpoint, ``from_quantized``).
"""

from __future__ import annotations

import math

import torch

from . import ops
from .ops import MetalNativeError
from .qformat import QuantizedWeight


class Linear:
    def __init__(self, in_features: int, out_features: int, bias: bool = True, device="cuda",
                 dtype: torch.dtype = torch.float16, generator: torch.Generator | None = None):
        self.in_features = in_features
        self.out_features = out_features
        limit = math.sqrt(6.0 / (in_features + out_features))   # Xavier uniform (linear.py:27-31)
        w = torch.rand((out_features, in_features), device=device, generator=generator, dtype=torch.float32)
        self.weight = ((w * 2.0 - 1.0) * limit).to(dtype)
        self.bias = torch.zeros(out_features, device=device, dtype=dtype) if bias else None

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        out = ops.matmul(x, self.weight, False, True)
        if self.bias is not None:
            out = out + self.bias
        return out

    def __repr__(self) -> str:
        return (f"Linear(in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None})")


class QuantizedLinear:
    def __init__(self, weight: QuantizedWeight):
        if weight.packed.device.type != "cuda":
            raise MetalNativeError("QuantizedLinear: weights must be GPU tensors")
        self.weight = weight
        self.in_features = weight.K
        self.out_features = weight.N
        if weight.bias is not None and (weight.bias.dtype != torch.float16 or weight.bias.numel() != weight.N):
            raise MetalNativeError("QuantizedLinear: bias must be Float16 [out_features]")

    @staticmethod
    def from_float(weight: torch.Tensor, bias: torch.Tensor | None = None, group_size: int = 128,
                   quant_type: str = "int4") -> "QuantizedLinear":
        """Quantize an fp16 ``[out_features, in_features]`` weight on the GPU."""
        w = weight.to(torch.float16)
        packed, scales, zeros = ops.quantize(w, group_size, quant_type)
        b = None if bias is None else bias.to(device=w.device, dtype=torch.float16).contiguous()
        return QuantizedLinear(QuantizedWeight(packed, scales, zeros, group_size, quant_type, w.shape[1], b))

    @staticmethod
    def from_quantized(weight: QuantizedWeight, device="cuda") -> "QuantizedLinear":
        return QuantizedLinear(weight.to(device))

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_features:
            raise MetalNativeError(f"QuantizedLinear: expected {self.in_features} input features, "
                                   f"got {x.shape[-1]}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype != torch.float16:
            x2 = x2.to(torch.float16)
        q = self.weight
        if q.bias is not None:
            y = ops.dequant_matmul(x2, q.packed, q.scales, q.zeros, q.group_size, q.quant_type,
                                   epilogue="bias", bias=q.bias)
        else:
            y = ops.dequant_matmul(x2, q.packed, q.scales, q.zeros, q.group_size, q.quant_type)
        return y.reshape(*lead, self.out_features)

    def dequantized_weight(self) -> torch.Tensor:
        """fp16 ``[out_features, in_features]`` (the fused kernels' dequant)."""
        q = self.weight
        return ops.dequantize(q.packed, q.scales, q.zeros, q.group_size, q.quant_type, K=q.K)

    def __repr__(self) -> str:
        q = self.weight
        return (f"QuantizedLinear(in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={q.bias is not None}, quant_type={q.quant_type!r}, group_size={q.group_size})")
