"""Write tests/golden/known_answers.npz: the reference's own known-answer cases
for the quantized-linear path, re-pinned with exact fp16 values.

The cases are the fixtures of tests/cpp/test_dequant_matmul.mm (the only test
of this path in the reference): shapes, input patterns, scales and zeros are
taken from there (line numbers below).  Expected values are computed here by
exact arithmetic that does not use numpy's float16 nor the oracle:
  * fp16 rounding is CPython's IEEE half packing (``struct.pack('<e')``,
    round-half-to-even) with overflow mapped to +-inf;
  * ``w = RNE(RNE((q-8)*s) - z)``: (q-8)*s and the subtraction of two fp16
    values are exact in binary64, so each step rounds exactly once;
  * ``C = sum_k a_k * w_k`` is accumulated exactly with fractions.Fraction and
    rounded once to binary64 (``C_exact``) and then to fp16 (``C_f16``).
Inputs are converted to fp16 with round-to-nearest-even; the reference test's
``fp32_to_fp16`` truncates instead (test_dequant_matmul.mm:241-259), so the
truncated activations are stored too (``A_trunc``) -- they differ only for
LargeMatrix's 0.3/0.7 values.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import os
import struct
from fractions import Fraction

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.npz")


def f16_bits(x: float) -> int:
    """IEEE binary16 bits of x, round-half-to-even, overflow -> inf."""
    if math.isnan(x):
        return 0x7E00
    try:
        return struct.unpack("<H", struct.pack("<e", x))[0]
    except OverflowError:
        return 0xFC00 if x < 0 else 0x7C00


def f16_val(bits: int) -> float:
    return struct.unpack("<e", struct.pack("<H", bits))[0]


def rne16(x: float) -> float:
    return f16_val(f16_bits(x))


def trunc16(f: float) -> float:
    """The reference test's fp32_to_fp16 (test_dequant_matmul.mm:241-259):
    mantissa truncation, tiny values flushed."""
    b = struct.unpack("<I", struct.pack("<f", f))[0]
    sign = (b & 0x80000000) >> 16
    exp = ((b & 0x7F800000) >> 23) - 127 + 15
    man = b & 0x007FFFFF
    if exp <= 0:
        if exp < -10:
            return f16_val(sign)
        man |= 0x00800000
        return f16_val(sign | (man >> (14 - exp)))
    if exp >= 31:
        return f16_val(sign | 0x7C00)
    return f16_val(sign | (exp << 10) | (man >> 13))


def pack_flat(vals):
    """pack_int4 of test_dequant_matmul.mm:104-116 (low nibble first)."""
    out = []
    for i in range(0, len(vals), 2):
        lo = vals[i] & 0x0F
        hi = (vals[i + 1] & 0x0F) if i + 1 < len(vals) else 0
        out.append(lo | (hi << 4))
    return out


def case(name, M, N, K, g, qtype, a_fn, b_fn, s_val, z_val=0.0):
    G = (K + g - 1) // g
    a_f = [a_fn(i) for i in range(M * K)]
    A = [rne16(v) for v in a_f]
    A_tr = [trunc16(v) for v in a_f]
    q = [b_fn(i) for i in range(N * K)]
    s = [rne16(s_val)] * (N * G)
    z = [rne16(z_val)] * (N * G)
    W = []
    for n in range(N):
        for k in range(K):
            qi = q[n * K + k]
            qv = (qi - 8) if qtype == "int4" else qi
            sc = s[n * G + k // g]
            zr = z[n * G + k // g]
            W.append(rne16(rne16(qv * sc) - zr))
    C_exact, C16 = [], []
    for m in range(M):
        for n in range(N):
            acc = Fraction(0)
            for k in range(K):
                acc += Fraction(A[m * K + k]) * Fraction(W[n * K + k])
            c = float(acc)
            C_exact.append(c)
            C16.append(f16_bits(c))
    if qtype == "int4":
        wp = np.array(pack_flat(q), dtype=np.uint8).reshape(N, K // 2)
    else:
        wp = np.array(q, dtype=np.int8).reshape(N, K)
    to16 = lambda xs, shape: np.array([f16_bits(x) for x in xs], dtype=np.uint16).reshape(shape)
    return {
        f"{name}/meta": np.array([M, N, K, g, 0 if qtype == "int4" else 1], dtype=np.int64),
        f"{name}/A": to16(A, (M, K)),
        f"{name}/A_trunc": to16(A_tr, (M, K)),
        f"{name}/Wp": wp,
        f"{name}/scales": to16(s, (N, G)),
        f"{name}/zeros": to16(z, (N, G)),
        f"{name}/W": to16(W, (N, K)),
        f"{name}/C_exact": np.array(C_exact, dtype=np.float64).reshape(M, N),
        f"{name}/C_f16": np.array(C16, dtype=np.uint16).reshape(M, N),
    }


def main():
    d = {}
    ka = [3, 5, 2, 7, 1, 4, 6, 2]
    ka8 = [10, 20, 30, 40, 5, 15, 25, 35]
    # tests/cpp/test_dequant_matmul.mm:269-336 (scales 0.1 / 0.2 per row)
    c = case("INT4_SmallKnownAnswer", 1, 2, 4, 32, "int4", lambda i: float(i + 1), lambda i: ka[i], 0.1)
    s = np.array([[f16_bits(0.1)], [f16_bits(0.2)]], dtype=np.uint16)
    c["INT4_SmallKnownAnswer/scales"] = s
    W = [rne16(rne16((ka[n * 4 + k] - 8) * f16_val(int(s[n, 0]))) - 0.0) for n in range(2) for k in range(4)]
    c["INT4_SmallKnownAnswer/W"] = np.array([f16_bits(x) for x in W], dtype=np.uint16).reshape(2, 4)
    Cs = [float(sum(Fraction(k + 1) * Fraction(W[n * 4 + k]) for k in range(4))) for n in range(2)]
    c["INT4_SmallKnownAnswer/C_exact"] = np.array(Cs).reshape(1, 2)
    c["INT4_SmallKnownAnswer/C_f16"] = np.array([f16_bits(x) for x in Cs], dtype=np.uint16).reshape(1, 2)
    d.update(c)
    # :338-398
    d.update(case("INT4_SquareMatrix", 16, 16, 32, 32, "int4", lambda i: (i % 7 - 3.0) * 0.5,
                  lambda i: i % 16, 0.05))
    # :400-439
    d.update(case("INT4_NonAlignedK", 4, 8, 48, 32, "int4", lambda i: 1.0, lambda i: 5, 0.1))
    # :441-479
    d.update(case("INT4_NonAlignedN", 4, 48, 32, 32, "int4", lambda i: 1.0, lambda i: 3, 0.1))
    # :481-526 (A uses float(i % 11 - 5) * 0.1f: an fp32 product, computed in fp32 here)
    f32 = lambda x: struct.unpack("<f", struct.pack("<f", x))[0]
    d.update(case("INT4_LargeMatrix", 64, 128, 256, 64, "int4",
                  lambda i: f32(f32(i % 11 - 5.0) * f32(0.1)), lambda i: i % 16, 0.05))
    # :528-566 and :568-606 (all M rows checked here)
    d.update(case("INT4_VecMat", 1, 64, 128, 32, "int4", lambda i: 0.5, lambda i: 4, 0.1))
    d.update(case("INT4_VecMatBatch", 4, 64, 128, 32, "int4", lambda i: 0.5, lambda i: 4, 0.1))
    # :612-649
    d.update(case("INT8_SmallKnownAnswer", 1, 2, 4, 32, "int8", lambda i: float(i + 1), lambda i: ka8[i], 0.1))
    # :651-705
    d.update(case("INT8_SquareMatrix", 16, 16, 32, 32, "int8", lambda i: (i % 7 - 3.0) * 0.5,
                  lambda i: i % 50 - 25, 0.05))
    # :707-746
    for g in (32, 64, 128):
        d.update(case(f"GroupSize_Variants_g{g}", 16, 32, 128, g, "int4", lambda i: 1.0, lambda i: 5, 0.1))
    # the zero term, which no reference test exercises (all their zeros are 0)
    d.update(case("INT4_NonzeroZero", 3, 16, 64, 32, "int4", lambda i: ((i * 37) % 13 - 6) * 0.25,
                  lambda i: (i * 7) % 16, 0.0123, z_val=-0.0456))
    d.update(case("INT8_NonzeroZero", 3, 16, 64, 32, "int8", lambda i: ((i * 37) % 13 - 6) * 0.25,
                  lambda i: (i * 29) % 255 - 127, 0.0031, z_val=0.0077))
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({len(d)} arrays)")


if __name__ == "__main__":
    main()
