"""mq_dequant_matmul_noalloc (the entry point that allocates nothing) against
mq_dequant_matmul, through the C ABI, on the split-K decode GEMV whose
partial sums it keeps in the library's fixed scratch array: bit-identical
outputs on two calls in a row, the second with a smaller input, and a clear
error for a shape beyond the scratch maximum."""

import numpy as np
import pytest
import torch

from oracle import mq_oracle as O

pytestmark = pytest.mark.gpu


def _call(lib, fn, x, wp, s, z, out, g, qt, M, N, K, stream):
    p = lambda t: t.data_ptr()
    return fn(p(x), K, p(wp), wp.stride(0) * wp.element_size(), p(s), p(z), p(out), N, M, N, K, g, qt, 0, None,
              None, 0, stream)


@pytest.fixture()
def forced_split_k(gpu):
    import metal_native as mn

    mn.set_option("force_path", 6)
    yield mn
    mn.set_option("force_path", 0)


def test_noalloc_matches_dequant_matmul(forced_split_k, gpu):
    mn = forced_split_k
    from metal_native import _lib

    lib = _lib.lib
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for M, K, N, g in ((8, 18944, 3584, 128), (3, 2048, 512, 64)):
        x, wp, s, z = O.make_int4_problem(M, K, N, g, seed=M + K)
        t = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in (x, wp, s, z)]
        ref = torch.empty((M, N), dtype=torch.float16, device=gpu)
        got = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
        assert _call(lib, lib.mq_dequant_matmul, *t, ref, g, 0, M, N, K, stream) == 0
        assert mn.last_path() == "decode"
        assert _call(lib, lib.mq_dequant_matmul_noalloc, *t, got, g, 0, M, N, K, stream) == 0, lib.mq_last_error()
        assert mn.last_path() == "decode"
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, K, N)
        yref = O.matmul_f32acc(x, O.dequant_int4(wp, s, z, K, g))
        err = np.abs(got.cpu().numpy().astype(np.float64) - yref)
        assert (err <= 1e-2 + 1e-3 * np.abs(yref)).all()


def test_noalloc_rejects_shapes_beyond_the_scratch(forced_split_k, gpu):
    from metal_native import _lib

    lib = _lib.lib
    stream = torch.cuda.current_stream(gpu).cuda_stream
    M, K, N, g = 16, 131072, 8192, 128   # split-K partials far above 8 MiB
    x = torch.zeros((M, K), dtype=torch.float16, device=gpu)
    wp = torch.zeros((N, K // 2), dtype=torch.uint8, device=gpu)
    s = torch.zeros((N, K // g), dtype=torch.float16, device=gpu)
    out = torch.zeros((M, N), dtype=torch.float16, device=gpu)
    rc = _call(lib, lib.mq_dequant_matmul_noalloc, x, wp, s, s, out, g, 0, M, N, K, stream)
    assert rc == 4 and b"fixed scratch" in lib.mq_last_error()


@pytest.mark.parametrize("M,K,N,g,want,ref_opts", [
    # M <= 4 with activations longer than LDS: the row-block plan would need
    # K parts (workspace), so the no-allocation entry point runs the split-K GEMV
    (4, 18944, 3584, 128, "decode", {"force_path": 6}),
    (1, 18944, 3584, 128, "rows", {}),
    # middle band: M = 5..16 takes the register-streamed GEMV (no workspace
    # either way), M > 16 the prefill GEMM without its K split (no workspace)
    (16, 18944, 3584, 128, "rstream", {}),
    (32, 18944, 3584, 128, "gemmw", {"gemm_split": 0}),
])
def test_noalloc_automatic_paths(gpu, M, K, N, g, want, ref_opts):
    """The automatic route of the no-allocation entry point: the kernel it
    takes where the allocating entry point would use a workspace, and outputs
    bit-identical to mq_dequant_matmul run on that same kernel."""
    import metal_native as mn
    from metal_native import _lib

    lib = _lib.lib
    stream = torch.cuda.current_stream(gpu).cuda_stream
    x, wp, s, z = O.make_int4_problem(M, K, N, g, seed=M + 7)
    t = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in (x, wp, s, z)]
    got = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    ref = torch.empty((M, N), dtype=torch.float16, device=gpu)
    assert _call(lib, lib.mq_dequant_matmul_noalloc, *t, got, g, 0, M, N, K, stream) == 0, lib.mq_last_error()
    assert mn.last_path() == want, mn.last_path()
    for k, v in ref_opts.items():
        mn.set_option(k, v)
    try:
        assert _call(lib, lib.mq_dequant_matmul, *t, ref, g, 0, M, N, K, stream) == 0, lib.mq_last_error()
        assert mn.last_path() == want, mn.last_path()
    finally:
        mn.set_option("force_path", 0)
        mn.set_option("gemm_split", 1)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), (M, K, N)
    yref = O.matmul_f32acc(x, O.dequant_int4(wp, s, z, K, g))
    err = np.abs(got.cpu().numpy().astype(np.float64) - yref)
    assert (err <= 1e-2 + 1e-3 * np.abs(yref)).all()
