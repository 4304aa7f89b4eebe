"""Pins the CPU oracle (oracle/mq_oracle.py) before it is trusted as the checker.

* the reference's known-answer cases (tests/golden/known_answers.npz, made by
  exact arithmetic in tests/golden/make_golden.py, not by the oracle);
* a brute-force sweep of the dequant formula over all nibbles / int8 values
  and a grid of fp16 scales and zeros (subnormal, normal, overflowing),
  against CPython's IEEE half rounding -- with a check that the sweep tells
  the two-rounding formula apart from a fused single rounding;
* closed forms: one-hot activations select dequantized weights exactly,
  linearity in A, row independence, SwiGLU against binary64 exp.
"""

import math
import os
import struct

import numpy as np
import pytest

from oracle import mq_oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "known_answers.npz")


def h(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


def rne16(x: float) -> float:
    try:
        return struct.unpack("<e", struct.pack("<e", x))[0]
    except OverflowError:
        return math.copysign(math.inf, x)


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def cases(gold):
    return sorted({k.split("/")[0] for k in gold.files})


def test_golden_file_has_all_reference_cases(gold):
    names = cases(gold)
    for want in ["INT4_SmallKnownAnswer", "INT4_SquareMatrix", "INT4_NonAlignedK", "INT4_NonAlignedN",
                 "INT4_LargeMatrix", "INT4_VecMat", "INT4_VecMatBatch", "INT8_SmallKnownAnswer",
                 "INT8_SquareMatrix", "GroupSize_Variants_g32", "GroupSize_Variants_g64",
                 "GroupSize_Variants_g128"]:
        assert want in names


def test_oracle_matches_goldens(gold):
    for name in cases(gold):
        M, N, K, g, qt = gold[f"{name}/meta"]
        qtype = "int4" if qt == 0 else "int8"
        A = h(gold[f"{name}/A"])
        wp = gold[f"{name}/Wp"]
        s, z = h(gold[f"{name}/scales"]), h(gold[f"{name}/zeros"])
        W = O.dequantize(wp, s, z, int(K), int(g), qtype)
        np.testing.assert_array_equal(W.view(np.uint16), gold[f"{name}/W"], err_msg=name)
        C = O.dequant_matmul(A, wp, s, z, int(g), qtype)
        ce = gold[f"{name}/C_exact"]
        err = np.abs(C.astype(np.float64) - ce)
        assert (err <= 1e-2 + 1e-3 * np.abs(ce)).all(), name
        # at most one fp16 ulp away from the exactly rounded result
        c16 = h(gold[f"{name}/C_f16"]).astype(np.float64)
        ulp = np.spacing(np.abs(c16).astype(np.float16)).astype(np.float64)
        assert (np.abs(C.astype(np.float64) - c16) <= ulp).all(), name


def test_reference_known_answer_assertions(gold):
    """The reference's own assertions: C = (-3.3, -9.0) +- 0.2
    (tests/cpp/test_dequant_matmul.mm:329-335)."""
    n = "INT4_SmallKnownAnswer"
    C = O.dequant_matmul(h(gold[f"{n}/A"]), gold[f"{n}/Wp"], h(gold[f"{n}/scales"]),
                         h(gold[f"{n}/zeros"]), 32, "int4").astype(np.float64)
    assert abs(C[0, 0] + 3.3) <= 0.2 and abs(C[0, 1] + 9.0) <= 0.2
    assert C[0, 0] != 0 and C[0, 1] != 0


def test_truncating_inputs_only_differ_in_large_matrix(gold):
    for name in cases(gold):
        same = np.array_equal(gold[f"{name}/A"], gold[f"{name}/A_trunc"])
        assert same == (name != "INT4_LargeMatrix"), name


# --------------------------------------------------------------------------
# brute-force dequant sweep
# --------------------------------------------------------------------------

SCALE_BITS = [0x0001, 0x0003, 0x00FF, 0x03FF, 0x0400, 0x1000, 0x2E66, 0x3266, 0x2148, 0x3C00, 0x3C01,
              0x4000, 0x47FF, 0x5BFF, 0x7000, 0x77FF, 0x7BFF, 0x8001, 0xAE66, 0xBC00, 0x0000, 0x8000]
ZERO_BITS = [0x0000, 0x8000, 0x0001, 0x2E66, 0xAE66, 0x3C00, 0xC500, 0x1234, 0x9234, 0x7BFF, 0xFBFF]


def _sweep(qvals, offset):
    s = h(SCALE_BITS)
    z = h(ZERO_BITS)
    got = O._deq(np.array(qvals)[:, None, None] - offset, s[None, :, None], z[None, None, :])
    for i, q in enumerate(qvals):
        for j, sv in enumerate(s):
            p = rne16((q - offset) * float(sv))
            for k, zv in enumerate(z):
                want = rne16(p - float(zv))
                g = float(got[i, j, k])
                if math.isnan(want):
                    assert math.isnan(g)
                else:
                    assert g == want and math.copysign(1, g) == math.copysign(1, want), (q, sv, zv)
    return got


def test_dequant_int4_bruteforce():
    _sweep(list(range(16)), 8)


def test_dequant_int8_bruteforce():
    _sweep(list(range(-128, 128)), 0)


def test_sweep_distinguishes_fused_rounding():
    """A contracted (single-rounding) dequant differs from the two-rounding one
    somewhere in the sweep, so the sweep would catch an FMA contraction."""
    s = h(SCALE_BITS).astype(np.float64)
    z = h(ZERO_BITS).astype(np.float64)
    diff = 0
    for q in range(16):
        for sv in s:
            for zv in z:
                if not (math.isfinite(sv) and math.isfinite(zv)):
                    continue
                two = rne16(rne16((q - 8) * sv) - zv)
                one = rne16((q - 8) * sv - zv)
                diff += (two != one) and not (math.isnan(two) and math.isnan(one))
    assert diff > 0


def test_pack_order_matches_reference_helper():
    # pack_int4 (test_dequant_matmul.mm:104-116): low nibble = even index
    q = np.array([[3, 5, 2, 7], [1, 4, 6, 2]], dtype=np.uint8)
    assert O.pack_int4(q).tolist() == [[0x53, 0x72], [0x41, 0x26]]
    r = np.random.default_rng(1).integers(0, 16, (7, 18), dtype=np.uint8)
    np.testing.assert_array_equal(O.unpack_int4(O.pack_int4(r), 18), r)


def test_flat_dequantize_semantics():
    rng = np.random.default_rng(2)
    N, K, g = 6, 64, 32
    wp = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s = rng.uniform(0.01, 0.1, (N, K // g)).astype(np.float16)
    flat = O.dequantize_flat(wp, s, N * K, g, "int4").reshape(N, K)
    np.testing.assert_array_equal(flat, O.dequant_int4(wp, s, None, K, g))
    # g not dividing K: flat index i // g crosses rows (dequantize_kernel.metal:44-51)
    K2, g2 = 6, 4
    wp2 = rng.integers(0, 256, (3, K2 // 2), dtype=np.uint8)
    s2 = rng.uniform(0.01, 0.1, (5,)).astype(np.float16)
    out = O.dequantize_flat(wp2, s2, 3 * K2, g2, "int4")
    nib = O.unpack_int4(wp2, K2).reshape(-1).astype(np.int64)
    for i in range(3 * K2):
        assert float(out[i]) == rne16((int(nib[i]) - 8) * float(s2[i // g2]))
    q8 = rng.integers(-128, 128, (3 * K2,), dtype=np.int16).astype(np.int8)
    out8 = O.dequantize_flat(q8, s2, 3 * K2, g2, "int8")
    for i in range(3 * K2):
        assert float(out8[i]) == rne16(int(q8[i]) * float(s2[i // g2]))


# --------------------------------------------------------------------------
# matmul closed forms
# --------------------------------------------------------------------------

def test_one_hot_selects_weights_exactly():
    x, wp, s, z = O.make_int4_problem(1, 256, 40, 64, seed=3)
    W = O.dequant_int4(wp, s, z, 256, 64)
    for k in (0, 1, 63, 64, 255):
        a = np.zeros((1, 256), np.float16)
        a[0, k] = 1
        np.testing.assert_array_equal(O.dequant_matmul(a, wp, s, z, 64, "int4")[0], W[:, k])


def test_linearity_and_row_independence():
    x, wp, s, z = O.make_int4_problem(4, 512, 48, 128, seed=4)
    full = O.matmul_f32acc(x, O.dequant_int4(wp, s, z, 512, 128))
    for m in range(4):
        row = O.matmul_f32acc(x[m:m + 1], O.dequant_int4(wp, s, z, 512, 128))
        np.testing.assert_allclose(row[0], full[m], rtol=1e-6, atol=1e-5)
    two = O.matmul_f32acc((x.astype(np.float32) * 2).astype(np.float16), O.dequant_int4(wp, s, z, 512, 128))
    np.testing.assert_allclose(two, 2 * full, rtol=1e-6, atol=1e-5)


def test_matmul_against_float64():
    x, q, s, z, g = O.make_int8_problem(3, 384, 70, seed=5)
    W = O.dequant_int8(q, s, z, 384, g).astype(np.float64)
    ref = x.astype(np.float64) @ W.T
    got = O.dequant_matmul(x, q, s, z, g, "int8").astype(np.float64)
    assert (np.abs(got - ref) <= 1e-2 + 1e-3 * np.abs(ref)).all()


def test_swiglu_closed_form():
    g = np.array([0.0, -0.0, 1.0, -1.0, 10.0, -10.0, 20.0, -20.0, 0.5, 65504.0, -65504.0], np.float16)
    u = np.array([1.0, 2.0, 3.0, -1.5, 0.25, 4.0, 1.0, 1.0, -2.0, 1.0, 1.0], np.float16)
    out = O.swiglu(g, u).astype(np.float64)
    for i in range(len(g)):
        gv, uv = float(g[i]), float(u[i])
        want = gv / (1.0 + math.exp(-gv)) * uv if gv > -700 else 0.0
        assert abs(out[i] - want) <= 1e-3 * abs(want) + 1e-6, (gv, uv, out[i], want)
    assert out[0] == 0.0


def test_epilogue_composition():
    x, wp, s, z = O.make_int4_problem(2, 128, 64, 32, seed=6)
    full = O.dequant_matmul(x, wp, s, z, 32, "int4")
    sw = O.dequant_matmul(x, wp, s, z, 32, "int4", epilogue="swiglu")
    np.testing.assert_array_equal(sw, O.swiglu(full[:, :32], full[:, 32:]))
    b = np.linspace(-1, 1, 64).astype(np.float16)
    acc = O.matmul_f32acc(x, O.dequant_int4(wp, s, z, 128, 32))
    np.testing.assert_array_equal(O.dequant_matmul(x, wp, s, z, 32, "int4", epilogue="bias", bias=b),
                                  (acc + b.astype(np.float32)).astype(np.float16))


def test_vecmat_oracle():
    rng = np.random.default_rng(7)
    a = rng.standard_normal((3, 300)).astype(np.float16)
    b = rng.standard_normal((300, 260)).astype(np.float16)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    for got in (O.vecmat_f16(a, b, False), O.vecmat_f16(a, np.ascontiguousarray(b.T), True)):
        assert (np.abs(got.astype(np.float64) - ref) <= 1e-2 + 1e-3 * np.abs(ref)).all()


# --------------------------------------------------------------------------
# quantizer (extension)
# --------------------------------------------------------------------------

def test_quantize_roundtrip_on_grid_int4():
    rng = np.random.default_rng(8)
    N, K, g = 8, 256, 64
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    q[:, ::g] = 0
    q[:, 1::g] = 15  # every group spans the full 0..15 range
    s = np.full((N, K // g), 2.0 ** -6, np.float16)
    zp = rng.integers(0, 16, (N, K // g))
    w = ((q.astype(np.float64) - np.repeat(zp, g, axis=1)) * 2.0 ** -6).astype(np.float16)
    bp, s2, z2 = O.quantize(w, g, "int4")
    np.testing.assert_array_equal(O.dequant_int4(bp, s2, z2, K, g), w)


def test_quantize_error_bound():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((16, 512)) * 0.05).astype(np.float16)
    for qt, levels in (("int4", 15), ("int8", 254)):
        bp, s, z = O.quantize(w, 128, qt)
        d = O.dequantize(bp, s, z, 512, 128, qt).astype(np.float64)
        step = np.repeat(s.astype(np.float64), 128, axis=1)
        assert (np.abs(d - w.astype(np.float64)) <= 0.5 * step + 1e-3).all(), qt
