"""On-disk packed format and GPTQ/AWQ converters for the quantized linear path.

The reference keeps quantized weights only in memory (``QuantWeightCache``,
src/memory/quant_weight_cache.mm:41-63) and has no file format or converter;
these are the next-row extensions its packed layout needs:

* ``QuantizedWeight``: one layer in the reference's storage format -- int4
  ``uint8 [N, K/2]`` (k = 2j low nibble, 2j+1 high nibble,
  shaders/matmul_dequant_kernel.metal:37-38) or int8 ``[N, K]``, fp16
  ``scales`` / ``zeros`` ``[N, ceil(K/g)]`` with ``w = half(q-8)*s - z``
  (int4) / ``half(q)*s - z`` (int8).
* ``save_quantized`` / ``load_quantized``: a safetensors file holding
  ``<name>.qweight``, ``<name>.scales``, ``<name>.zeros`` (and
  ``<name>.bias``) with the group size, quant type and K per layer in the
  header metadata.  Loading goes through safetensors only (no pickle).
* ``from_gptq`` / ``from_awq``: repack 4-bit GPTQ / AWQ checkpoints, whose
  dequant is ``(q - zp) * s``, into the reference's ``(q - 8) * s - z``
  form with ``z = half((zp - 8) * s)``.  The nibbles are copied exactly; the
  weights they decode to differ from ``(q - zp) * s`` by the rounding of
  ``z`` (within one fp16 ulp of the weight, see the tests).

The converters are integer repacking in torch ops on the tensors' own device
(a load-time step, not the hot path); the numpy restatement they are tested
against is ``oracle.mq_oracle.gptq_to_reference`` / ``awq_to_reference``.
"""

from __future__ import annotations

import json
from dataclasses import dataclass

import torch

from .ops import MetalNativeError

FORMAT = "metal-native-amd/quantized-linear/1"
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)   # nibble j of an AWQ int32 holds column 8c + AWQ_ORDER[j]


@dataclass
class QuantizedWeight:
    packed: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    group_size: int
    quant_type: str
    K: int
    bias: torch.Tensor | None = None

    @property
    def N(self) -> int:
        return self.packed.shape[0]

    def to(self, device) -> "QuantizedWeight":
        mv = lambda t: None if t is None else t.to(device)
        return QuantizedWeight(mv(self.packed), mv(self.scales), mv(self.zeros), self.group_size, self.quant_type,
                               self.K, mv(self.bias))


def _check_layer(name: str, q: QuantizedWeight) -> None:
    if q.quant_type not in ("int4", "int8"):
        raise MetalNativeError(f"save_quantized: {name}: quant_type must be 'int4' or 'int8'")
    cols = q.K // 2 if q.quant_type == "int4" else q.K
    G = (q.K + q.group_size - 1) // q.group_size
    if tuple(q.packed.shape) != (q.N, cols):
        raise MetalNativeError(f"save_quantized: {name}: packed weights must be [N, {cols}]")
    for t, what in ((q.scales, "scales"), (q.zeros, "zeros")):
        if t.dtype != torch.float16 or tuple(t.shape) != (q.N, G):
            raise MetalNativeError(f"save_quantized: {name}: {what} must be Float16 [N, {G}]")


def save_quantized(path: str, layers: dict[str, QuantizedWeight]) -> None:
    from safetensors.torch import save_file

    tensors, meta = {}, {"format": FORMAT}
    for name, q in layers.items():
        _check_layer(name, q)
        tensors[f"{name}.qweight"] = q.packed.detach().contiguous().cpu()
        tensors[f"{name}.scales"] = q.scales.detach().contiguous().cpu()
        tensors[f"{name}.zeros"] = q.zeros.detach().contiguous().cpu()
        if q.bias is not None:
            tensors[f"{name}.bias"] = q.bias.detach().contiguous().cpu()
        meta[name] = json.dumps({"quant_type": q.quant_type, "group_size": q.group_size, "K": q.K})
    save_file(tensors, path, metadata=meta)


def load_quantized(path: str, device="cpu") -> dict[str, QuantizedWeight]:
    from safetensors import safe_open

    out = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise MetalNativeError(f"load_quantized: {path} is not a {FORMAT} file")
        keys = set(f.keys())
        for name, info in meta.items():
            if name == "format":
                continue
            d = json.loads(info)
            get = lambda suffix: f.get_tensor(f"{name}.{suffix}").to(device)
            bias = get("bias") if f"{name}.bias" in keys else None
            q = QuantizedWeight(get("qweight"), get("scales"), get("zeros"), int(d["group_size"]),
                                d["quant_type"], int(d["K"]), bias)
            _check_layer(name, q)
            out[name] = q
    return out


def _nibbles_of(words: torch.Tensor) -> torch.Tensor:
    """int32 [..., C] -> uint8 [..., C, 8] (nibble j from bits 4j..4j+3)."""
    shifts = torch.arange(0, 32, 4, device=words.device, dtype=torch.int32)
    return ((words[..., None] >> shifts) & 0xF).to(torch.uint8)


def _reference_zeros(zp: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """``half((zp - 8) * s)``: one fp32 product, one rounding."""
    return ((zp.to(torch.float32) - 8.0) * scales.to(torch.float32)).to(torch.float16)


def _pack_k(q: torch.Tensor) -> torch.Tensor:
    """uint8 nibbles [N, K] -> [N, K/2], k = 2j low nibble, 2j+1 high nibble."""
    return (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()


def from_gptq(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int,
              g_idx: torch.Tensor | None = None, zero_offset: int = 1, bias: torch.Tensor | None = None
              ) -> QuantizedWeight:
    """4-bit GPTQ (AutoGPTQ layout): ``qweight`` int32 ``[K/8, N]`` (word
    ``(i, n)`` holds k = 8i+j at bits 4j), ``qzeros`` int32 ``[G, N/8]``
    (word ``(gi, c)`` holds the zero point of column 8c+j at bits 4j, stored
    minus ``zero_offset``: 1 in the original format), ``scales`` fp16
    ``[G, N]``; dequant ``(q - zp) * s``.  Act-order checkpoints (a
    ``g_idx`` that is not ``k // group_size``) have no contiguous-group form
    and are refused."""
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise MetalNativeError("from_gptq: qweight and qzeros must be int32")
    K8, N = qweight.shape
    K = K8 * 8
    G = (K + group_size - 1) // group_size
    if tuple(qzeros.shape) != (G, (N + 7) // 8) or tuple(scales.shape) != (G, N):
        raise MetalNativeError("from_gptq: qzeros must be [G, N/8] and scales [G, N]")
    if g_idx is not None:
        want = torch.arange(K, device=g_idx.device) // group_size
        if not torch.equal(g_idx.to(torch.int64), want):
            raise MetalNativeError("from_gptq: act-order (g_idx) checkpoints are not supported")
    q = _nibbles_of(qweight.t().contiguous()).reshape(N, K)              # [N, K]
    zp = _nibbles_of(qzeros).reshape(G, -1)[:, :N].to(torch.int32) + zero_offset  # [G, N]
    s = scales.to(torch.float16)
    return QuantizedWeight(_pack_k(q), s.t().contiguous(), _reference_zeros(zp, s).t().contiguous(), group_size,
                           "int4", K, bias)


def from_awq(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int,
             bias: torch.Tensor | None = None) -> QuantizedWeight:
    """4-bit AWQ (GEMM layout): ``qweight`` int32 ``[K, N/8]`` and ``qzeros``
    int32 ``[G, N/8]``, nibble j of word c holding column ``8c + AWQ_ORDER[j]``;
    ``scales`` fp16 ``[G, N]``; dequant ``(q - zp) * s``."""
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise MetalNativeError("from_awq: qweight and qzeros must be int32")
    K, N8 = qweight.shape
    N = N8 * 8
    G = (K + group_size - 1) // group_size
    if tuple(qzeros.shape) != (G, N8) or tuple(scales.shape) != (G, N):
        raise MetalNativeError("from_awq: qzeros must be [G, N/8] and scales [G, N]")
    order = torch.tensor(AWQ_ORDER, device=qweight.device)
    inv = torch.argsort(order)   # column t of a word lives in nibble inv[t]

    def unscramble(words):
        nib = _nibbles_of(words)                    # [R, N/8, 8] by nibble
        return nib[:, :, inv].reshape(words.shape[0], N)

    q = unscramble(qweight).t().contiguous()        # [N, K]
    zp = unscramble(qzeros).to(torch.int32)         # [G, N]
    s = scales.to(torch.float16)
    return QuantizedWeight(_pack_k(q), s.t().contiguous(), _reference_zeros(zp, s).t().contiguous(), group_size,
                           "int4", K, bias)
