"""On-disk format and GPTQ/AWQ converters (host-side; the GPU use of the
converted weights is in test_gpu_parity.py)."""

import numpy as np
import pytest
import torch

import metal_native as mn
from metal_native import qformat as QF
from oracle import mq_oracle as O


def to_i32(words) -> np.ndarray:
    """Python ints (0 .. 2^32-1) -> int32 bit patterns."""
    return np.array(words, dtype=np.uint64).astype(np.uint32).view(np.int32)


def loop_pack_gptq(q, zp, offset=1):
    """Independent (loop) packer of the AutoGPTQ layout for tiny cases."""
    N, K = q.shape
    G = zp.shape[0]
    qw = [[0] * N for _ in range(K // 8)]
    for i in range(K // 8):
        for n in range(N):
            for j in range(8):
                qw[i][n] |= int(q[n, 8 * i + j]) << (4 * j)
    qz = [[0] * ((N + 7) // 8) for _ in range(G)]
    for gi in range(G):
        for n in range(N):
            qz[gi][n // 8] |= (int(zp[gi, n]) - offset) << (4 * (n % 8))
    return to_i32(qw), to_i32(qz)


def loop_pack_awq(q, zp):
    N, K = q.shape
    G = zp.shape[0]
    qw = [[0] * (N // 8) for _ in range(K)]
    for k in range(K):
        for c in range(N // 8):
            for j in range(8):
                qw[k][c] |= int(q[8 * c + O.AWQ_ORDER[j], k]) << (4 * j)
    qz = [[0] * (N // 8) for _ in range(G)]
    for gi in range(G):
        for c in range(N // 8):
            for j in range(8):
                qz[gi][c] |= int(zp[gi, 8 * c + O.AWQ_ORDER[j]]) << (4 * j)
    return to_i32(qw), to_i32(qz)


def problem(N, K, g, seed, zp_lo=0, zp_hi=16):
    rng = np.random.default_rng(seed)
    G = (K + g - 1) // g
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    zp = rng.integers(zp_lo, zp_hi, size=(G, N))
    s = rng.uniform(0.002, 0.03, size=(G, N)).astype(np.float16)
    return q, zp, s


def test_gptq_oracle_pinned_by_loop_packer():
    q, zp, s = problem(16, 64, 32, 0, zp_lo=1, zp_hi=17)   # stored zp - 1 in 0..15
    qw, qz = loop_pack_gptq(q, zp)
    bp, ss, zz = O.gptq_to_reference(qw, qz, s, 32)
    np.testing.assert_array_equal(O.unpack_int4(bp, 64), q)
    np.testing.assert_array_equal(ss, s.T)
    np.testing.assert_array_equal(zz, ((zp - 8.0) * s.astype(np.float32)).astype(np.float16).T)


def test_awq_oracle_pinned_by_loop_packer():
    q, zp, s = problem(16, 64, 32, 1)
    qw, qz = loop_pack_awq(q, zp)
    bp, ss, zz = O.awq_to_reference(qw, qz, s, 32)
    np.testing.assert_array_equal(O.unpack_int4(bp, 64), q)
    np.testing.assert_array_equal(zz, ((zp - 8.0) * s.astype(np.float32)).astype(np.float16).T)


@pytest.mark.parametrize("N,K,g", [(16, 64, 32), (24, 256, 128), (40, 128, 64)])
def test_converters_match_oracle(N, K, g):
    q, zp, s = problem(N, K, g, N + K, zp_lo=1, zp_hi=17)
    qw, qz = loop_pack_gptq(q, zp)
    got = QF.from_gptq(torch.from_numpy(qw), torch.from_numpy(qz), torch.from_numpy(s), g)
    want = O.gptq_to_reference(qw, qz, s, g)
    for a, b in zip((got.packed, got.scales, got.zeros), want):
        np.testing.assert_array_equal(a.numpy().view(np.uint8), b.view(np.uint8))
    q, zp, s = problem(N, K, g, N + K + 1)
    qw, qz = loop_pack_awq(q, zp)
    got = QF.from_awq(torch.from_numpy(qw), torch.from_numpy(qz), torch.from_numpy(s), g)
    want = O.awq_to_reference(qw, qz, s, g)
    for a, b in zip((got.packed, got.scales, got.zeros), want):
        np.testing.assert_array_equal(a.numpy().view(np.uint8), b.view(np.uint8))


def test_converted_weights_decode_close_to_the_checkpoint():
    """The reference form w = half(half(q-8)*s) - half((zp-8)*s) against the
    checkpoint's half((q-zp)*s): four roundings apart, two of terms up to 8s
    and two of the result, so within ulp(8s) + ulp(w)."""
    N, K, g = 64, 512, 128
    q, zp, s = problem(N, K, g, 7)
    qw, qz = loop_pack_awq(q, zp)
    bp, ss, zz = O.awq_to_reference(qw, qz, s, g)
    ref_form = O.dequant_int4(bp, ss, zz, K, g).astype(np.float32)
    ckpt = O.dequant_zero_point(q, zp.T, s.T, g).astype(np.float32)
    s8 = (8.0 * O._expand_groups(ss, K, g).astype(np.float32)).astype(np.float16)
    ulp = lambda v: np.spacing(np.abs(v).astype(np.float16)).astype(np.float32)
    bound = ulp(s8) + ulp(ckpt)
    err = np.abs(ref_form - ckpt)
    assert np.all(err <= bound), float((err / bound).max())
    assert err.mean() < 0.5 * bound.mean()   # most weights are (nearly) exact


def test_gptq_refuses_act_order():
    q, zp, s = problem(16, 64, 32, 3, zp_lo=1, zp_hi=17)
    qw, qz = loop_pack_gptq(q, zp)
    g_idx = torch.arange(64).flip(0) // 32
    with pytest.raises(mn.MetalNativeError, match="act-order"):
        QF.from_gptq(torch.from_numpy(qw), torch.from_numpy(qz), torch.from_numpy(s), 32, g_idx=g_idx)


def test_save_load_roundtrip(tmp_path):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((32, 256)) * 0.05).astype(np.float16)
    bp, s, z = O.quantize(w, 64, "int4")
    layers = {
        "blk0.down": QF.QuantizedWeight(torch.from_numpy(bp), torch.from_numpy(s), torch.from_numpy(z), 64, "int4",
                                        256, torch.from_numpy(w[:, 0].copy())),
    }
    q8, s8, z8 = O.quantize(w, 256, "int8")
    layers["blk0.gate"] = QF.QuantizedWeight(torch.from_numpy(q8), torch.from_numpy(s8), torch.from_numpy(z8),
                                             256, "int8", 256)
    path = str(tmp_path / "m.safetensors")
    QF.save_quantized(path, layers)
    back = QF.load_quantized(path)
    assert set(back) == set(layers)
    for name, a in layers.items():
        b = back[name]
        assert (b.group_size, b.quant_type, b.K) == (a.group_size, a.quant_type, a.K)
        for x, y in ((a.packed, b.packed), (a.scales, b.scales), (a.zeros, b.zeros)):
            assert torch.equal(x, y)
        assert (a.bias is None) == (b.bias is None)
        if a.bias is not None:
            assert torch.equal(a.bias, b.bias)


def test_load_refuses_foreign_files(tmp_path):
    from safetensors.torch import save_file

    path = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(2)}, path, metadata={"format": "pt"})
    with pytest.raises(mn.MetalNativeError, match="not a"):
        QF.load_quantized(path)


def test_save_checks_shapes(tmp_path):
    bad = QF.QuantizedWeight(torch.zeros(4, 10, dtype=torch.uint8), torch.zeros(4, 1, dtype=torch.float16),
                             torch.zeros(4, 1, dtype=torch.float16), 32, "int4", 32)
    with pytest.raises(mn.MetalNativeError, match="packed weights"):
        QF.save_quantized(str(tmp_path / "b.safetensors"), {"l": bad})
