"""QuantWeightCache and the Linear layers (the next rows after the kernels)."""

import numpy as np
import pytest
import torch

from oracle import mq_oracle as O

TOL_ABS, TOL_REL = 1e-2, 1e-3


def close(y, ref, what):
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    bad = err > TOL_ABS + TOL_REL * np.abs(ref.astype(np.float64))
    assert not bad.any(), f"{what}: {bad.sum()} outside tolerance, max err {err.max():.3g}"


# ---------------------------------------------------------------------------
# host-only: bookkeeping
# ---------------------------------------------------------------------------

def test_cache_accounting_and_errors():
    import metal_native as mn

    c = mn.QuantWeightCache()
    c.register_weight("a", torch.zeros(8, 32, dtype=torch.uint8), torch.zeros(8, 2, dtype=torch.float16), "int4")
    c.register_weight("b", torch.zeros(4, 64, dtype=torch.int8), torch.zeros(4, 1, dtype=torch.float16), "int8")
    # quant_weight_cache.mm:177-196: int4 0.5 B/element, int8 1 B, scales 2 B each
    assert c.total_footprint() == (8 * 64) // 2 + 16 * 2 + 4 * 64 + 4 * 2
    assert c.dequantized_footprint() == 0
    with pytest.raises(mn.MetalNativeError, match="not registered"):
        c.get_dequantized("zzz")
    with pytest.raises(mn.MetalNativeError, match="divide"):
        c.register_weight("c", torch.zeros(3, 5, dtype=torch.int8), torch.zeros(4, dtype=torch.float16), "int8")


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.gpu
@pytest.mark.parametrize("qt", ["int4", "int8"])
def test_cache_dequantizes_like_the_standalone_kernels(gpu, qt):
    import metal_native as mn

    rng = np.random.default_rng(2)
    N, K, g = 48, 256, 64
    if qt == "int4":
        qb = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    else:
        qb = rng.integers(-127, 128, size=(N, K), dtype=np.int16).astype(np.int8)
    s = rng.uniform(0.001, 0.02, size=(N * K // g,)).astype(np.float16)
    c = mn.QuantWeightCache()
    c.register_weight("w", torch.from_numpy(qb).to(gpu), torch.from_numpy(s).to(gpu), qt)
    d1 = c.get_dequantized("w")
    torch.cuda.synchronize()
    want = O.dequantize_flat(qb, s, N * K, g, qt).reshape(N, K)
    np.testing.assert_array_equal(d1.cpu().numpy().view(np.uint16), want.view(np.uint16))
    assert tuple(d1.shape) == (N, K)
    assert c.get_dequantized("w") is d1                       # cached
    assert c.dequantized_footprint() == N * K * 2
    c.evict_dequantized()
    assert c.dequantized_footprint() == 0
    small = mn.QuantWeightCache(budget_bytes=16)
    small.register_weight("w", torch.from_numpy(qb).to(gpu), torch.from_numpy(s).to(gpu), qt)
    small.get_dequantized("w")
    assert small.dequantized_footprint() == 0                 # over budget: not kept


@pytest.mark.gpu
@pytest.mark.parametrize("qt,g", [("int4", 128), ("int4", 64), ("int8", 128)])
@pytest.mark.parametrize("lead", [(1,), (5,), (2, 32), (130,)])
def test_quantized_linear(gpu, qt, g, lead):
    import metal_native as mn

    rng = np.random.default_rng(len(lead) + lead[-1])
    K, N = 512, 384
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    lin = mn.nn.QuantizedLinear.from_float(torch.from_numpy(w).to(gpu), torch.from_numpy(b).to(gpu), g, qt)
    x = rng.standard_normal((*lead, K)).astype(np.float16)
    y = lin(torch.from_numpy(x).to(gpu))
    assert tuple(y.shape) == (*lead, N)
    bp, s, z = O.quantize(w, g, qt)
    Wd = O.dequantize(bp, s, z, K, g, qt)
    ref = O.matmul_f32acc(x.reshape(-1, K), Wd) + b.astype(np.float32)
    close(y.reshape(-1, N).cpu().numpy(), ref, f"QuantizedLinear {qt} g{g} {lead}")
    np.testing.assert_array_equal(lin.dequantized_weight().cpu().numpy().view(np.uint16), Wd.view(np.uint16))


@pytest.mark.gpu
def test_quantized_linear_from_checkpoint_file(gpu, tmp_path):
    import metal_native as mn
    from metal_native import qformat as QF

    rng = np.random.default_rng(9)
    w = (rng.standard_normal((256, 1024)) * 0.05).astype(np.float16)
    lin = mn.nn.QuantizedLinear.from_float(torch.from_numpy(w).to(gpu), None, 128, "int4")
    path = str(tmp_path / "l.safetensors")
    QF.save_quantized(path, {"proj": lin.weight})
    lin2 = mn.nn.QuantizedLinear.from_quantized(QF.load_quantized(path)["proj"], gpu)
    x = torch.from_numpy(rng.standard_normal((3, 1024)).astype(np.float16)).to(gpu)
    assert torch.equal(lin(x), lin2(x))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4, 8, 40])
def test_linear_fp16(gpu, M):
    import metal_native as mn

    gen = torch.Generator(device=gpu)
    gen.manual_seed(M)
    lin = mn.nn.Linear(512, 320, bias=True, device=gpu, generator=gen)
    lin.bias = torch.randn(320, device=gpu, generator=gen).half()
    x = torch.randn((M, 512), device=gpu, generator=gen).half()
    y = lin(x)
    ref = (x.float() @ lin.weight.float().t()).half().float() + lin.bias.float()
    close(y.float().cpu().numpy(), ref.cpu().numpy(), f"Linear M={M}")
