"""CPU checks of the C-ABI library: it loads, exports exactly what
include/metal_native_amd.h declares, and rejects bad arguments before touching
a GPU (validation mirrors src/ops/matmul.mm:910-934)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "metal_native_amd.h")


def declared():
    text = open(HEADER).read()
    return re.findall(r"MQ_API\s+[\w\s\*]+?\b(mq_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def lib():
    from metal_native import _lib

    return _lib.lib


def test_header_declares_entry_points():
    names = declared()
    for want in ["mq_dequant_matmul", "mq_dequantize", "mq_quantize", "mq_vecmat_f16", "mq_swiglu_f16",
                 "mq_last_error"]:
        assert want in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared():
        assert hasattr(lib, name), name
    from metal_native import _lib

    assert set(declared()) == set(_lib.SIGNATURES)


def test_abi_version_and_error_strings(lib):
    assert lib.mq_abi_version() == 3
    assert lib.mq_error_to_string(0) == b"Success"
    assert lib.mq_error_to_string(4) == b"InvalidArgument"
    assert lib.mq_error_to_string(8) == b"NotImplemented"


def test_validation_without_gpu(lib):
    P = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    call = lambda M, N, K, g, qt, epi, ldw=None, res=None, ldr=0: lib.mq_dequant_matmul(
        P, K, P, (K // 2 if qt == 0 else K) if ldw is None else ldw, P, P, P, N, M, N, K, g, qt, epi,
        None, res, ldr, None)
    assert call(0, 8, 32, 32, 0, 0) == 4
    assert b"positive" in lib.mq_last_error()
    assert call(1, 8, 33, 32, 0, 0) == 4  # odd K for int4
    assert b"INT4 weights must be [N, K/2]" in lib.mq_last_error()
    assert call(1, 8, 32, 32, 0, 0, ldw=8) == 4
    assert b"INT4 weights must be [N, K/2]" in lib.mq_last_error()
    assert call(1, 8, 32, 32, 1, 0, ldw=16) == 4
    assert b"INT8 weights must be [N, K]" in lib.mq_last_error()
    assert call(1, 7, 32, 32, 0, 5) == 4  # SwiGLU needs even N
    assert call(1, 8, 32, 32, 5, 0) == 4
    for epi in (1, 2, 3):  # bias, bias+ReLU, bias+SiLU without bias
        assert call(1, 8, 32, 32, 0, epi) == 4
        assert b"bias" in lib.mq_last_error()
    assert call(1, 8, 32, 32, 0, 4) == 4  # residual epilogue without residual
    assert b"residual" in lib.mq_last_error()
    assert call(1, 8, 32, 32, 0, 4, res=P, ldr=7) == 4  # ldr < N
    assert b"ldr" in lib.mq_last_error()
    assert call(2, 8, 32, 32, 0, 4, res=P, ldr=16) == 4  # residual aliasing the output with another stride
    assert b"ldr == ldc" in lib.mq_last_error()
    assert call(1, 8, 32, 32, 0, 6) == 4
    assert b"unknown epilogue" in lib.mq_last_error()
    assert lib.mq_dequantize(P, 16, P, P, P, 32, 4, 32, 32, 0, 1, None) == 4  # flat + zeros
    assert lib.mq_swiglu_f16(None, P, P, 10, None) == 4
    assert lib.mq_vecmat_f16(P, 10, P, 10, P, 10, 1, 300, 300, 1, None) == 4  # lda < K


def test_set_option(lib):
    assert lib.mq_set_option(b"force_path", 9) == 4
    assert lib.mq_set_option(b"force_path", 1) == 4  # retired path id
    assert lib.mq_set_option(b"gemv_steps", 9) == 4
    assert lib.mq_set_option(b"gemv_tiles_per_wg", 3) == 4
    assert lib.mq_set_option(b"nonsense", 1) == 4
    assert b"unknown key" in lib.mq_last_error()
    assert lib.mq_set_option(b"gemm_impl", 3) == 4
    assert lib.mq_set_option(b"gemm_impl", 2) == 0
    assert lib.mq_set_option(b"gemm_impl", 0) == 0
    assert lib.mq_set_option(b"force_path", 0) == 0


def test_python_surface_mirrors_reference():
    import metal_native as mn

    for name in ("dequant_matmul", "matmul", "synchronize", "MetalNativeError"):
        assert hasattr(mn._C, name)
    assert callable(mn._C.fast.swiglu)
    assert issubclass(mn.MetalNativeError, RuntimeError)
    from metal_native.ops import quant_type_code

    # bindings/bind_ops.cpp:373: "int4" -> INT4, anything else -> INT8
    assert quant_type_code("int4") == 0 and quant_type_code("int8") == 1 and quant_type_code("x") == 1


def test_python_rejects_cpu_tensors():
    import torch

    import metal_native as mn

    a = torch.zeros(1, 64, dtype=torch.float16)
    with pytest.raises(mn.MetalNativeError, match="GPU tensor"):
        mn.dequant_matmul(a, torch.zeros(8, 32, dtype=torch.uint8), torch.zeros(8, 2, dtype=torch.float16),
                          torch.zeros(8, 2, dtype=torch.float16), 32, "int4")


def test_quantize_needs_a_gpu_tensor():
    """The quantizer runs on the library's kernel only: CPU tensors are refused."""
    import torch

    import metal_native as mn

    with pytest.raises(mn.MetalNativeError, match="GPU tensor"):
        mn.quantize(torch.zeros(4, 64, dtype=torch.float16), 32, "int4")


def test_rowmajor_copies_overlapping_rows():
    """A broadcast or overlapping view (row stride below the row length) is
    handed to the kernels as a contiguous copy, never with a row stride that
    would read past its storage; ordinary row-major views keep their stride."""
    import torch

    from metal_native.ops import _rowmajor

    x = torch.arange(8, dtype=torch.float16).reshape(1, 8)
    e = x.expand(64, 8)                       # stride (0, 1)
    t, ld = _rowmajor(e, "activations", "op")
    assert ld == 8 and t.is_contiguous() and t.shape == (64, 8)
    assert torch.equal(t, e)
    base = torch.arange(64, dtype=torch.float16)
    o = base.as_strided((10, 8), (4, 1))      # rows overlap by half
    t, ld = _rowmajor(o, "activations", "op")
    assert ld == 8 and torch.equal(t, o)
    big = torch.zeros(16, 24, dtype=torch.float16)
    v = big[:, :8]                            # row stride 24 >= 8: kept
    t, ld = _rowmajor(v, "activations", "op")
    assert ld == 24 and t.data_ptr() == v.data_ptr()
    one = big[3:4, :8]                        # a single row: stride unused
    t, ld = _rowmajor(one, "activations", "op")
    assert ld == 8 and t.data_ptr() == one.data_ptr()
    col = big[:, :8].t()                      # strided last dimension: copied
    t, ld = _rowmajor(col, "activations", "op")
    assert t.is_contiguous() and ld == 16


def test_decode_loop_refuses_positions_past_the_cache():
    """The decode benchmark checks on the host that every position it will
    write lies inside the KV cache."""
    import types

    import pytest as _pt

    from metal_native.decoder import DecoderConfig, decode_tokens_per_second

    model = types.SimpleNamespace(prefilled=512, cfg=DecoderConfig(max_len=576), device=None)
    with _pt.raises(ValueError, match="exceed the KV cache"):
        decode_tokens_per_second(model, n_tokens=65)
