"""``QuantWeightCache``: quantized weights with optional dequantized fp16 copies.

Mirrors include/metal_native/memory/quant_weight_cache.h:22-50 and
src/memory/quant_weight_cache.mm:41-196:

* ``register_weight(name, quantized, scales, format)`` (:41-63): keeps the
  tensors (borrowed), derives ``num_elements`` (INT4: two per byte) and
  ``group_size = num_elements / scales.numel()``; re-registering a name
  replaces it (insert_or_assign).
* ``get_dequantized(name)`` (:65-153): the cached fp16 copy if there is one,
  else dequantizes with the standalone kernels' semantics -- flat element
  index, group ``i // group_size``, no zero term
  (shaders/dequantize_kernel.metal:9-163) -- into a tensor of the quantized
  shape with the last dimension doubled for INT4 (:81-90), and keeps it when
  the memory budget allows (:145-149).  Unknown names raise
  ``MetalNativeError("quant_weight_cache: weight not registered")`` (:69-71).
* ``evict_dequantized()`` (:155-160), ``dequantized_footprint()`` and
  ``total_footprint()`` (:162-196) with the reference's byte accounting.

The dequantization is the library's kernel (``mq_dequantize``, flat mode);
this class is bookkeeping.  The reference consults a process-wide
MemoryBudgetController (cache only while its pressure multiplier is >= 0.5);
here the budget is explicit: a copy is kept while the dequantized copies
stay within ``budget_bytes`` (None = unlimited).  Device memory comes from
the torch allocator, so a returned tensor stays valid after eviction.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass

import torch

from . import ops
from .ops import MetalNativeError

INT8 = "int8"   # QuantFormat::INT8 (quant_weight_cache.h:17-20)
INT4 = "int4"   # QuantFormat::INT4


@dataclass
class _Entry:
    quantized: torch.Tensor
    scales: torch.Tensor
    dequantized: torch.Tensor | None
    fmt: str
    num_elements: int
    group_size: int


class QuantWeightCache:
    def __init__(self, budget_bytes: int | None = None):
        self._mu = threading.Lock()
        self._weights: dict[str, _Entry] = {}
        self.budget_bytes = budget_bytes

    def register_weight(self, name: str, quantized: torch.Tensor, scales: torch.Tensor, fmt: str) -> None:
        if fmt not in (INT4, INT8):
            raise MetalNativeError("quant_weight_cache: format must be 'int4' or 'int8'")
        n = quantized.numel() * (2 if fmt == INT4 else 1)
        if scales.numel() == 0 or n % scales.numel():
            raise MetalNativeError("quant_weight_cache: scales must divide the element count")
        with self._mu:
            self._weights[name] = _Entry(quantized, scales, None, fmt, n, n // scales.numel())

    def get_dequantized(self, name: str) -> torch.Tensor:
        with self._mu:
            e = self._weights.get(name)
            if e is None:
                raise MetalNativeError("quant_weight_cache: weight not registered")
            if e.dequantized is not None:
                return e.dequantized
            shape = list(e.quantized.shape)
            if e.fmt == INT4:
                shape[-1] *= 2
            flat = e.quantized.reshape(1, -1)
            K = e.num_elements
            out = ops.dequantize(flat, e.scales.reshape(-1), None, e.group_size, e.fmt, K=K, flat_groups=True)
            out = out.reshape(shape)
            used = sum(x.num_elements * 2 for x in self._weights.values() if x.dequantized is not None)
            if self.budget_bytes is None or used + e.num_elements * 2 <= self.budget_bytes:
                e.dequantized = out
            return out

    def evict_dequantized(self) -> None:
        with self._mu:
            for e in self._weights.values():
                e.dequantized = None

    def dequantized_footprint(self) -> int:
        with self._mu:
            return sum(e.num_elements * 2 for e in self._weights.values() if e.dequantized is not None)

    def total_footprint(self) -> int:
        with self._mu:
            total = 0
            for e in self._weights.values():
                total += e.num_elements if e.fmt == INT8 else e.num_elements // 2
                total += e.scales.numel() * 2
                if e.dequantized is not None:
                    total += e.num_elements * 2
            return total
