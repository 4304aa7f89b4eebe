"""CPU restatement of MetalNative's quantized-weight linear path (numpy).

TEST INFRASTRUCTURE ONLY.  This module is the checker for the HIP kernels in
``metal-native_amd``.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and there only to check or
to time the CPU baseline -- never as the computation that is shipped or
measured as the product.

Every function cites the reference source it restates (paths are relative to
the reference tree, kimsejun0629/metal-native).

Semantics restated
------------------
* int4 storage: ``Bp`` is ``uint8 [N, K/2]``; byte ``j`` of row ``n`` holds
  ``k = 2j`` in the low nibble and ``k = 2j+1`` in the high nibble
  (shaders/matmul_dequant_kernel.metal:37-38,129-139;
  tests/cpp/test_dequant_matmul.mm:104-116).
* int8 storage: ``int8 [N, K]`` (matmul_dequant_kernel.metal:400-412).
* per-group fp16 ``scales`` / ``zeros``: ``[N, ceil(K/g)]`` row-major, group of
  element ``k`` is ``k // g`` (matmul_dequant_kernel.metal:98,141-143).
* dequant: ``w = half(q - 8) * scale - zero`` (int4) and
  ``w = half(q) * scale - zero`` (int8), i.e. two IEEE fp16 round-to-nearest-even
  operations, multiply first (matmul_dequant_kernel.metal:42-43,47-49).  The
  reference's own CPU oracle uses the same order
  (tests/cpp/test_dequant_matmul.mm:149,180).
* standalone dequantize: no zero term and a *flat* group index ``i // g``
  over the ``N*K`` elements (shaders/dequantize_kernel.metal:9-54).
* matmul: ``C[M,N] = A[M,K] . W[N,K]^T`` with fp16 products accumulated in fp32
  and one final rounding to fp16 (matmul_dequant_kernel.metal:88,217;
  matmul_reference at tests/cpp/test_dequant_matmul.mm:191-213).
* SwiGLU: ``half(silu(float(g)) * float(u))`` with ``silu(v) = v / (1+exp(-v))``
  applied to the fp16 outputs of the projection
  (shaders/fused_swiglu.metal:48-84; src/future/future_stubs.mm:61-101).
* fused epilogues on the fp32 accumulator, one rounding after
  (shaders/matmul_fused_epilogue.metal:97-124): bias ``half(acc + float(b[n]))``,
  bias+ReLU ``half(max(acc + b, 0))``, bias+SiLU ``half(v / (1 + exp(-v)))``,
  residual ``half(acc + float(r[m, n]))``.

Why fp32-then-round equals fp16 arithmetic: for one +, - or x of two fp16
values the exact result rounded to fp32 (p=24 >= 2*11+2) and then to fp16 is
the same as rounding the exact result to fp16 directly (double rounding is
innocuous; Figueroa, "When is double rounding innocuous?", SIGNUM 1995).
"""

from __future__ import annotations

import numpy as np

INT4 = "int4"
INT8 = "int8"


# --------------------------------------------------------------------------
# packing
# --------------------------------------------------------------------------

def pack_int4(q: np.ndarray) -> np.ndarray:
    """Pack nibbles ``q`` (uint8 0..15, shape [N, K], K even) into [N, K/2].

    Low nibble = even k, high nibble = odd k
    (tests/cpp/test_dequant_matmul.mm:104-116).
    """
    q = np.asarray(q, dtype=np.uint8)
    if q.ndim != 2 or q.shape[1] % 2:
        raise ValueError("pack_int4 expects [N, K] with even K")
    if (q > 15).any():
        raise ValueError("int4 values must be in 0..15")
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)


def unpack_int4(bp: np.ndarray, K: int) -> np.ndarray:
    """Inverse of :func:`pack_int4` (matmul_dequant_kernel.metal:37-38)."""
    bp = np.asarray(bp, dtype=np.uint8)
    out = np.empty((bp.shape[0], bp.shape[1] * 2), dtype=np.uint8)
    out[:, 0::2] = bp & 0x0F
    out[:, 1::2] = bp >> 4
    return out[:, :K]


# --------------------------------------------------------------------------
# dequantization
# --------------------------------------------------------------------------

def _expand_groups(t: np.ndarray, K: int, g: int) -> np.ndarray:
    """Broadcast a [N, ceil(K/g)] per-group tensor to [N, K] (group = k // g)."""
    t = np.asarray(t, dtype=np.float16)
    G = (K + g - 1) // g
    if t.ndim != 2 or t.shape[1] != G:
        raise ValueError(f"expected [N, {G}] per-group tensor, got {t.shape}")
    return np.repeat(t, g, axis=1)[:, :K]


def _deq(qf: np.ndarray, s: np.ndarray, z) -> np.ndarray:
    """``half(half(qf) * s) - z`` with each op rounded to fp16 (RNE)."""
    with np.errstate(over="ignore", invalid="ignore"):
        p = (qf.astype(np.float32) * s.astype(np.float32)).astype(np.float16)
        if z is None:
            return p
        return (p.astype(np.float32) - z.astype(np.float32)).astype(np.float16)


def dequant_int4(bp, scales, zeros, K: int, g: int) -> np.ndarray:
    """fp16 [N, K] weights of the fused int4 path.

    Restates ``unpack_int4_pair`` (shaders/matmul_dequant_kernel.metal:29-44)
    with the B-tile indexing of :128-162.  ``zeros=None`` drops the zero term.
    """
    q = unpack_int4(bp, K).astype(np.int16) - 8
    s = _expand_groups(scales, K, g)
    z = None if zeros is None else _expand_groups(zeros, K, g)
    return _deq(q, s, z)


def dequant_int8(bq, scales, zeros, K: int, g: int) -> np.ndarray:
    """fp16 [N, K] weights of the fused int8 path
    (``dequant_int8``, shaders/matmul_dequant_kernel.metal:47-49,400-412)."""
    q = np.asarray(bq, dtype=np.int8)[:, :K].astype(np.int16)
    s = _expand_groups(scales, K, g)
    z = None if zeros is None else _expand_groups(zeros, K, g)
    return _deq(q, s, z)


def dequantize(bp, scales, zeros, K: int, g: int, quant_type: str) -> np.ndarray:
    if quant_type == INT4:
        return dequant_int4(bp, scales, zeros, K, g)
    return dequant_int8(bp, scales, zeros, K, g)


def dequantize_flat(packed, scales, num_elements: int, g: int, quant_type: str) -> np.ndarray:
    """Standalone kernels: flat group index ``i // g`` and no zero term.

    int4: ``out[i] = half(nib_i - 8) * scales[i // g]``
    (shaders/dequantize_kernel.metal:26-54, vec variant :100-163).
    int8: ``out[i] = half(q_i) * scales[i // g]`` (:9-22, vec :58-96).
    """
    packed = np.asarray(packed).reshape(-1)
    scales = np.asarray(scales, dtype=np.float16).reshape(-1)
    if quant_type == INT4:
        b = packed.astype(np.uint8)
        q = np.empty(b.size * 2, dtype=np.int16)
        q[0::2] = b & 0x0F
        q[1::2] = b >> 4
        q = q[:num_elements] - 8
    else:
        q = packed.view(np.int8)[:num_elements].astype(np.int16)
    s = scales[np.arange(num_elements) // g]
    return _deq(q, s, None)


# --------------------------------------------------------------------------
# matmul + epilogues
# --------------------------------------------------------------------------

def silu_f32(v: np.ndarray) -> np.ndarray:
    """``v / (1 + exp(-v))`` in fp32 (shaders/fused_swiglu.metal:67,
    matmul_fused_epilogue.metal:116)."""
    v = v.astype(np.float32)
    with np.errstate(over="ignore"):
        return (v / (np.float32(1.0) + np.exp(-v))).astype(np.float32)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``fused_swiglu_fp16`` (shaders/fused_swiglu.metal:48-84)."""
    g = np.asarray(gate, dtype=np.float16).astype(np.float32)
    u = np.asarray(up, dtype=np.float16).astype(np.float32)
    return (silu_f32(g) * u).astype(np.float16)


def matmul_f32acc(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """fp32-accumulated ``A . W^T`` of fp16 operands, result in fp32.

    Restates ``matmul_reference`` (tests/cpp/test_dequant_matmul.mm:191-213);
    fp16 x fp16 products are exact in fp32.
    """
    return np.asarray(a, np.float16).astype(np.float32) @ np.asarray(w, np.float16).astype(np.float32).T


def apply_epilogue(acc: np.ndarray, epilogue: str | None, bias=None, residual=None) -> np.ndarray:
    """Round the fp32 accumulator to fp16 after the optional epilogue.

    * ``None``   -> ``half(acc)`` (matmul_dequant_kernel.metal:217)
    * ``"bias"`` -> ``half(acc + float(bias[n]))`` (matmul_fused_epilogue.metal:108-110)
    * ``"bias_relu"`` -> ``half(max(0, acc + float(bias[n])))`` (:111-113)
    * ``"bias_silu"`` -> ``half(v / (1 + exp(-v)))``, ``v = acc + float(bias[n])`` (:114-117)
    * ``"residual"`` -> ``half(acc + float(residual[m, n]))`` (:118-121)
    * ``"swiglu"`` -> columns ``[0,F)`` are gate, ``[F,2F)`` up; the projection
      is rounded to fp16 first and then ``fused_swiglu_fp16`` is applied,
      which is the reference's two-dispatch composition
      ``fast.swiglu(dequant_matmul(...))`` (fused_swiglu.metal:48-84).
    """
    if epilogue is None or epilogue == "none":
        return acc.astype(np.float16)
    if epilogue in ("bias", "bias_relu", "bias_silu"):
        v = (acc + np.asarray(bias, np.float16).astype(np.float32)[None, :]).astype(np.float32)
        if epilogue == "bias_relu":
            v = np.maximum(v, np.float32(0.0))
        elif epilogue == "bias_silu":
            v = silu_f32(v)
        return v.astype(np.float16)
    if epilogue == "residual":
        return (acc + np.asarray(residual, np.float16).astype(np.float32)).astype(np.float16)
    if epilogue == "swiglu":
        F = acc.shape[1] // 2
        h = acc.astype(np.float16)
        return swiglu(h[:, :F], h[:, F:])
    raise ValueError(f"unknown epilogue {epilogue!r}")


def dequant_matmul(a, bp, scales, zeros, group_size: int, quant_type: str,
                   epilogue: str | None = None, bias=None, residual=None) -> np.ndarray:
    """``_C.dequant_matmul`` semantics (bindings/bind_ops.cpp:366-382 ->
    src/ops/matmul.mm:903-1029 -> shaders/matmul_dequant_kernel.metal),
    for *every* row of A (the reference's M<=8 kernel writes only row 0; the
    documented contract ``C = A . deq(W)^T`` is restated here instead).
    """
    a = np.asarray(a, dtype=np.float16)
    K = a.shape[1]
    w = dequantize(bp, scales, zeros, K, group_size, quant_type)
    return apply_epilogue(matmul_f32acc(a, w), epilogue, bias, residual)


def vecmat_f16(a, b, transpose_b: bool) -> np.ndarray:
    """fp16 GEMV route of ``_C.matmul`` for M<=8: ``C = A @ op(B)`` with fp32
    accumulation and fp16 output (shaders/matmul_vecmat_kernel.metal:59-139;
    API contract include/metal_native/ops/matmul.h:18-37)."""
    a = np.asarray(a, np.float16).astype(np.float32)
    b = np.asarray(b, np.float16).astype(np.float32)
    return (a @ (b.T if transpose_b else b)).astype(np.float16)


# --------------------------------------------------------------------------
# quantizer (extension: the reference has no quantize op)
# --------------------------------------------------------------------------

def quantize(w: np.ndarray, group_size: int, quant_type: str):
    """Quantize fp16 ``W [N, K]`` into the reference's storage format.

    No reference function exists (nothing in the reference calls a quantizer);
    this is the inverse of the dequant formula above.
    int4 (asymmetric): per group ``s = (max-min)/15``, integer zero-point
    ``zp = clamp(round(-min/s), 0, 15)``, ``q = clamp(round(w/s) + zp, 0, 15)``
    and the reference-signature zero ``zeros = half((zp - 8) * s)`` so that
    ``(q-8)*s - zeros ~= (q - zp) * s``.
    int8 (symmetric): ``s = max|w| / 127``, ``q = clamp(round(w/s), -127, 127)``,
    ``zeros = 0``.
    """
    w = np.asarray(w, dtype=np.float16).astype(np.float32)
    N, K = w.shape
    g = group_size
    G = (K + g - 1) // g
    pad = G * g - K
    wp = np.pad(w, ((0, 0), (0, pad)), mode="edge").reshape(N, G, g)
    if quant_type == INT4:
        lo = wp.min(axis=2)
        hi = wp.max(axis=2)
        s = ((hi - lo) / 15.0).astype(np.float16)
        s = np.where(s == 0, np.float16(1.0), s)
        sf = s.astype(np.float32)
        zp = np.clip(np.rint(-lo / sf), 0, 15)
        q = np.clip(np.rint(wp / sf[:, :, None]) + zp[:, :, None], 0, 15).astype(np.uint8)
        q = q.reshape(N, G * g)[:, :K]
        zeros = ((zp - 8.0) * sf).astype(np.float16)
        return pack_int4(q), s, zeros
    amax = np.abs(wp).max(axis=2)
    s = (amax / 127.0).astype(np.float16)
    s = np.where(s == 0, np.float16(1.0), s)
    q = np.clip(np.rint(wp / s.astype(np.float32)[:, :, None]), -127, 127).astype(np.int8)
    return q.reshape(N, G * g)[:, :K].copy(), s, np.zeros_like(s)


# --------------------------------------------------------------------------
# seeded synthetic inputs (the workloads the benchmark names)
# --------------------------------------------------------------------------

def make_int4_problem(M: int, K: int, N: int, g: int, seed: int = 0):
    """int4 inputs: nibbles U{0..15}, scales U(0.005, 0.02), integer zero-points
    U{0..15} mapped to the reference signature as ``zeros = half((zp-8)*s)``,
    x ~ N(0, 1); all fp16."""
    rng = np.random.default_rng(seed)
    G = (K + g - 1) // g
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s = rng.uniform(0.005, 0.02, size=(N, G)).astype(np.float16)
    zp = rng.integers(0, 16, size=(N, G)).astype(np.float32)
    z = ((zp - 8.0) * s.astype(np.float32)).astype(np.float16)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    return x, pack_int4(q), s, z


def make_int8_problem(M: int, K: int, N: int, seed: int = 0, g: int | None = None):
    """int8 symmetric per-output-channel inputs: q U{-127..127}, per-column
    scales U(0.001, 0.01), zeros 0, x ~ N(0,1).  ``g=None`` means one group
    spanning K (shape [N, 1])."""
    rng = np.random.default_rng(seed)
    gg = K if g is None else g
    G = (K + gg - 1) // gg
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int16).astype(np.int8)
    s_col = rng.uniform(0.001, 0.01, size=(N, 1)).astype(np.float16)
    s = np.repeat(s_col, G, axis=1)
    z = np.zeros_like(s)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    return x, q, s, z, gg


# --------------------------------------------------------------------------
# GPTQ / AWQ checkpoints -> the reference's storage format
# --------------------------------------------------------------------------
# Neither format appears in the reference; they are the two common 4-bit
# checkpoint layouts (AutoGPTQ's original "gptq" format and AutoAWQ's GEMM
# format), restated from their published packing rules:
#   GPTQ: qweight int32 [K/8, N], word (i, n) holds q[n, 8i + j] at bits 4j;
#         qzeros int32 [G, N/8], word (g, c) holds zp[g, 8c + j] - 1 at bits 4j;
#         scales fp16 [G, N]; w = (q - zp) * s.
#   AWQ:  qweight int32 [K, N/8], word (k, c) holds q[8c + ORDER[j], k] at bits 4j
#         with ORDER = (0, 2, 4, 6, 1, 3, 5, 7); qzeros int32 [G, N/8] likewise
#         (no offset); scales fp16 [G, N]; w = (q - zp) * s.
# The reference form keeps q and sets zeros = half((zp - 8) * s).

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def _words_to_nibbles(words: np.ndarray) -> np.ndarray:
    u = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    return np.stack([(u >> (4 * j)) & 0xF for j in range(8)], axis=-1).astype(np.uint8)


def gptq_to_reference(qweight, qzeros, scales, g: int, zero_offset: int = 1):
    """-> (Bp uint8 [N, K/2], scales fp16 [N, G], zeros fp16 [N, G])."""
    K8, N = qweight.shape
    K = 8 * K8
    q = _words_to_nibbles(qweight).transpose(1, 0, 2).reshape(N, K)        # [N, K]
    zp = _words_to_nibbles(qzeros).reshape(qzeros.shape[0], -1)[:, :N].astype(np.int32) + zero_offset
    s = np.asarray(scales, dtype=np.float16)
    z = ((zp.astype(np.float32) - 8.0) * s.astype(np.float32)).astype(np.float16)
    return pack_int4(q), s.T.copy(), z.T.copy()


def awq_to_reference(qweight, qzeros, scales, g: int):
    K, N8 = qweight.shape
    N = 8 * N8
    inv = np.argsort(np.asarray(AWQ_ORDER))
    q = _words_to_nibbles(qweight)[:, :, inv].reshape(K, N).T              # [N, K]
    zp = _words_to_nibbles(qzeros)[:, :, inv].reshape(qzeros.shape[0], N).astype(np.int32)
    s = np.asarray(scales, dtype=np.float16)
    z = ((zp.astype(np.float32) - 8.0) * s.astype(np.float32)).astype(np.float16)
    return pack_int4(np.ascontiguousarray(q)), s.T.copy(), z.T.copy()


def dequant_zero_point(q, zp, scales, g: int) -> np.ndarray:
    """The checkpoints' own dequant ``(q - zp) * s`` in fp32 then one fp16
    rounding: q uint8 [N, K], zp int [N, G], scales fp16 [N, G]."""
    K = q.shape[1]
    return ((q.astype(np.float32) - _expand_groups(zp.astype(np.float32), K, g))
            * _expand_groups(np.asarray(scales, np.float16).astype(np.float32), K, g)).astype(np.float16)
