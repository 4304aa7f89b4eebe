"""Python-facing ops of the quantized-linear path on PyTorch-ROCm tensors.

Names, argument order, ``quant_type`` string handling and error texts follow
the reference's pybind11 surface:
  * ``dequant_matmul``  -- bindings/bind_ops.cpp:366-382 -> src/ops/matmul.mm:903-1029
  * ``matmul``          -- bindings/bind_ops.cpp:170-183 -> src/ops/matmul.mm:599-882
                           (the M<=8 vecmat route, select_kernel :167-190)
  * ``fast.swiglu``     -- bindings/bind_ops.cpp:84-93 -> src/future/future_stubs.mm:61-101
  * ``MetalNativeError``-- bindings/bind_core.cpp:347 (MNException translation)
Extensions (no reference counterpart): ``dequantize`` (the dequantize kernels
are only reachable through QuantWeightCache in the reference,
src/memory/quant_weight_cache.mm:65-153), ``quantize``, and the ``epilogue`` /
``bias`` keywords of ``dequant_matmul``.

Every op launches a HIP kernel of libmetal_native_amd.so on the current torch
stream and returns without synchronising, like the reference's lazy command
buffers.  Outputs are fresh tensors owned by the caller.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_L = _lib.lib


class MetalNativeError(RuntimeError):
    """Mirror of ``_C.MetalNativeError`` (bindings/bind_core.cpp:347).

    ``code`` carries the MetalNativeError number
    (include/metal_native/core/error.h:21-31)."""

    def __init__(self, message: str, code: int = _lib.INVALID_ARGUMENT):
        super().__init__(message)
        self.code = code


def _check(rc: int) -> None:
    if rc != _lib.SUCCESS:
        msg = _L.mq_last_error().decode()
        name = _L.mq_error_to_string(rc).decode()
        raise MetalNativeError(f"{msg} [{name}]", rc)


def _invalid(msg: str):
    raise MetalNativeError(msg, _lib.INVALID_ARGUMENT)


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require_cuda(t: torch.Tensor, what: str, op: str):
    if not isinstance(t, torch.Tensor):
        _invalid(f"{op}: {what} must be a torch.Tensor")
    if t.device.type != "cuda":
        _invalid(f"{op}: {what} must be a GPU tensor (got {t.device})")


def _rowmajor(t: torch.Tensor, what: str, op: str) -> tuple[torch.Tensor, int]:
    """``(t', ld)``: a 2-D tensor whose rows the kernels can address as
    ``base + i * ld`` with unit stride along the last dimension, and that
    row stride in elements.  A tensor whose rows overlap or alias (a
    broadcast ``expand``, an ``as_strided`` view with ``stride(0) < size(1)``)
    or whose last dimension is strided is copied to a contiguous tensor
    first, so a kernel never reads past the storage it was given."""
    if t.dim() != 2:
        _invalid(f"{op}: {what} must be 2D")
    rows, cols = t.shape
    if (cols > 1 and t.stride(1) != 1) or (rows > 1 and t.stride(0) < cols):
        t = t.contiguous()
    return t, (t.stride(0) if rows > 1 else cols)


# ---------------------------------------------------------------------------
# dequant_matmul
# ---------------------------------------------------------------------------

_EPILOGUES = {None: _lib.EPILOGUE_NONE, "none": _lib.EPILOGUE_NONE,
              "bias": _lib.EPILOGUE_BIAS, "bias_relu": _lib.EPILOGUE_BIAS_RELU,
              "bias_silu": _lib.EPILOGUE_BIAS_SILU, "residual": _lib.EPILOGUE_RESIDUAL,
              "swiglu": _lib.EPILOGUE_SWIGLU}
_BIAS_EPILOGUES = (_lib.EPILOGUE_BIAS, _lib.EPILOGUE_BIAS_RELU, _lib.EPILOGUE_BIAS_SILU)


def quant_type_code(quant_type: str) -> int:
    """``"int4"`` selects INT4; any other string selects INT8, as in
    bindings/bind_ops.cpp:373."""
    return _lib.QUANT_INT4 if quant_type == "int4" else _lib.QUANT_INT8


def dequant_matmul(activations: torch.Tensor, weights_packed: torch.Tensor, scales: torch.Tensor,
                   zeros: torch.Tensor, group_size: int, quant_type: str, *,
                   epilogue: str | None = None, bias: torch.Tensor | None = None,
                   residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused dequantize + matmul: ``activations[M,K] . deq(weights)[N,K]^T`` -> fp16 ``[M,N]``.

    Validation and messages follow src/ops/matmul.mm:910-934.  Beyond the
    reference, the dtype/shape/device of weights, scales and zeros are checked
    too (the reference reads out of bounds on a mismatch), and
    ``group_size == K`` (one group per row: per-output-channel scales) is
    accepted as an extension.
    Epilogues (fp32, before the one fp16 rounding; the reference's
    MatmulEpilogue set, include/metal_native/ops/fused_matmul.h:18-24):
    ``"bias"`` adds ``bias[N]``, ``"bias_relu"`` / ``"bias_silu"`` then apply
    ReLU / SiLU, ``"residual"`` adds ``residual[M, N]`` (which may be ``out``
    itself, for an in-place residual add).  ``epilogue="swiglu"`` treats
    weight rows ``[0,N/2)`` as gate and ``[N/2,N)`` as up and returns
    ``[M, N/2] = fast.swiglu(gate, up)`` of the fp16 projection.  ``out``
    (extension): an fp16 ``[M, N_out]`` tensor with unit column stride to
    write instead of a new one.
    """
    op = "dequant_matmul"
    _require_cuda(activations, "activations", op)
    if activations.dim() != 2:
        _invalid("dequant_matmul: activations must be 2D [M, K]")
    if activations.dtype != torch.float16:
        _invalid("dequant_matmul: activations must be Float16")
    M, K = activations.shape
    if group_size not in (32, 64, 128) and group_size != K:
        _invalid("dequant_matmul: group_size must be 32, 64, or 128")
    qt = quant_type_code(quant_type)
    for t, what in ((weights_packed, "weights_packed"), (scales, "scales"), (zeros, "zeros")):
        _require_cuda(t, what, op)
        if t.device != activations.device:
            _invalid(f"{op}: {what} must be on the activations' device")
    if weights_packed.dim() != 2:
        _invalid(f"{op}: weights_packed must be 2D")
    N = weights_packed.shape[0]
    if qt == _lib.QUANT_INT4:
        if weights_packed.shape[1] != K // 2:
            _invalid("dequant_matmul: INT4 weights must be [N, K/2]")
        if K % 2:
            _invalid("dequant_matmul: INT4 weights must be [N, K/2] with K even")
        if weights_packed.dtype not in (torch.uint8, torch.int8):
            _invalid(f"{op}: INT4 weights must be uint8 (two nibbles per byte)")
    else:
        if weights_packed.shape[1] != K:
            _invalid("dequant_matmul: INT8 weights must be [N, K]")
        if weights_packed.dtype not in (torch.int8, torch.uint8):
            _invalid(f"{op}: INT8 weights must be int8")
    G = (K + group_size - 1) // group_size
    for t, what in ((scales, "scales"), (zeros, "zeros")):
        if t.dtype != torch.float16:
            _invalid(f"{op}: {what} must be Float16")
        if tuple(t.shape) != (N, G):
            _invalid(f"{op}: {what} must be [N, ceil(K/group_size)] = [{N}, {G}], got {list(t.shape)}")
    if epilogue not in _EPILOGUES:
        _invalid(f"{op}: unknown epilogue {epilogue!r}")
    epi = _EPILOGUES[epilogue]
    if epi in _BIAS_EPILOGUES:
        if bias is None:
            _invalid(f"{op}: epilogue={epilogue!r} needs bias")
        _require_cuda(bias, "bias", op)
        if bias.dtype != torch.float16 or bias.numel() != N:
            _invalid(f"{op}: bias must be Float16 [N]")
        bias = bias.contiguous()
    elif bias is not None:
        _invalid(f"{op}: bias given without a bias epilogue")
    if epi == _lib.EPILOGUE_RESIDUAL:
        if residual is None:
            _invalid(f"{op}: epilogue='residual' needs residual")
        _require_cuda(residual, "residual", op)
        if residual.dtype != torch.float16 or tuple(residual.shape) != (M, N):
            _invalid(f"{op}: residual must be Float16 [M, N] = [{M}, {N}]")
    elif residual is not None:
        _invalid(f"{op}: residual given without epilogue='residual'")
    if epi == _lib.EPILOGUE_SWIGLU and N % 2:
        _invalid(f"{op}: SwiGLU needs an even number of weight rows")
    n_out = N // 2 if epi == _lib.EPILOGUE_SWIGLU else N

    activations, lda = _rowmajor(activations, "activations", op)
    weights_packed, ldw = _rowmajor(weights_packed, "weights_packed", op)
    scales = scales.contiguous()
    zeros = zeros.contiguous()
    dev = activations.device
    if out is None:
        out = torch.empty((M, n_out), dtype=torch.float16, device=dev)
    else:
        _require_cuda(out, "out", op)
        if out.dtype != torch.float16 or tuple(out.shape) != (M, n_out) or (n_out > 1 and out.stride(1) != 1) \
                or (M > 1 and out.stride(0) < n_out):
            _invalid(f"{op}: out must be Float16 [{M}, {n_out}] with unit column stride")
    ldc = out.stride(0) if M > 1 else n_out
    ldr = 0
    if residual is not None:
        if residual.data_ptr() == out.data_ptr():
            if residual.stride() != out.stride():
                _invalid(f"{op}: a residual that is the output must have the output's strides")
            ldr = ldc
        else:
            residual, ldr = _rowmajor(residual, "residual", op)
    if M == 0 or n_out == 0:
        return out
    with torch.cuda.device(dev):
        rc = _L.mq_dequant_matmul(
            _ptr(activations), lda, _ptr(weights_packed), ldw, _ptr(scales), _ptr(zeros), _ptr(out),
            ldc, M, N, K, group_size, qt, epi, _ptr(bias), _ptr(residual), ldr, _stream_handle(dev))
    _check(rc)
    return out


# ---------------------------------------------------------------------------
# dequantize (extension)
# ---------------------------------------------------------------------------

def dequantize(weights_packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None,
               group_size: int, quant_type: str, *, K: int | None = None,
               flat_groups: bool = False) -> torch.Tensor:
    """fp16 ``[N, K]`` weights.

    ``flat_groups=False``: the fused kernels' dequant, ``half(q-8)*s[n,k/g] - z[n,k/g]``
    (shaders/matmul_dequant_kernel.metal:29-49,128-162); ``zeros=None`` drops
    the zero term.
    ``flat_groups=True``: the standalone kernels' semantics,
    ``out.flat[i] = half(q_i - 8) * scales.flat[i // g]`` with no zero
    (shaders/dequantize_kernel.metal:9-163 as dispatched by
    src/memory/quant_weight_cache.mm:96-140); the output has the INT4 packed
    shape with its last dimension doubled, as there (:81-90).
    """
    op = "dequantize"
    _require_cuda(weights_packed, "weights_packed", op)
    qt = quant_type_code(quant_type)
    if weights_packed.dim() != 2:
        _invalid(f"{op}: weights_packed must be 2D")
    N, cols = weights_packed.shape
    if K is None:
        K = cols * 2 if qt == _lib.QUANT_INT4 else cols
    if qt == _lib.QUANT_INT4 and cols != K // 2:
        _invalid("dequantize: INT4 weights must be [N, K/2]")
    if qt == _lib.QUANT_INT8 and cols != K:
        _invalid("dequantize: INT8 weights must be [N, K]")
    if group_size < 1:
        _invalid(f"{op}: group_size must be positive")
    _require_cuda(scales, "scales", op)
    if scales.dtype != torch.float16:
        _invalid(f"{op}: scales must be Float16")
    if flat_groups:
        if zeros is not None:
            _invalid(f"{op}: flat groups take no zeros")
        weights_packed = weights_packed.contiguous()
        need = (N * K + group_size - 1) // group_size
        if scales.numel() < need:
            _invalid(f"{op}: scales must hold ceil(N*K/group_size) = {need} values")
    else:
        G = (K + group_size - 1) // group_size
        if tuple(scales.shape) != (N, G):
            _invalid(f"{op}: scales must be [N, ceil(K/group_size)] = [{N}, {G}]")
        if zeros is not None:
            _require_cuda(zeros, "zeros", op)
            if zeros.dtype != torch.float16 or tuple(zeros.shape) != (N, G):
                _invalid(f"{op}: zeros must be Float16 [N, ceil(K/group_size)]")
            zeros = zeros.contiguous()
    scales = scales.contiguous()
    weights_packed, ldw = _rowmajor(weights_packed, "weights_packed", op)
    dev = weights_packed.device
    out = torch.empty((N, K), dtype=torch.float16, device=dev)
    if N == 0 or K == 0:
        return out
    with torch.cuda.device(dev):
        rc = _L.mq_dequantize(_ptr(weights_packed), ldw, _ptr(scales), _ptr(zeros), _ptr(out), K, N, K,
                              group_size, qt, 1 if flat_groups else 0, _stream_handle(dev))
    _check(rc)
    return out


# ---------------------------------------------------------------------------
# quantize (extension; the reference has no quantizer)
# ---------------------------------------------------------------------------

def quantize(w: torch.Tensor, group_size: int, quant_type: str):
    """Quantize fp16 ``W [N, K]`` (GPU tensor) into ``(weights_packed, scales,
    zeros)`` of the reference's storage format; the exact inverse of the
    dequant formula on weights that lie on the quantization grid.

    int4 (asymmetric, per group): ``s = half((max-min)/15)``,
    ``zp = clamp(rint(-min/s), 0, 15)``, ``q = clamp(rint(w/s)+zp, 0, 15)``,
    ``zeros = half((zp-8)*s)``, so ``(q-8)*s - zeros ~= (q-zp)*s``.
    int8 (symmetric, per group): ``s = half(max|w|/127)``,
    ``q = clamp(rint(w/s), -127, 127)``, ``zeros = 0``.
    Runs the library's quantize kernel (``mq_quantize``).
    """
    op = "quantize"
    _require_cuda(w, "weights", op)
    if w.dim() != 2:
        _invalid("quantize: weights must be 2D [N, K]")
    if w.dtype != torch.float16:
        _invalid("quantize: weights must be Float16")
    N, K = w.shape
    qt = quant_type_code(quant_type)
    if qt == _lib.QUANT_INT4 and (K % 2 or group_size % 2):
        _invalid("quantize: INT4 needs an even K and an even group_size")
    if group_size < 1:
        _invalid("quantize: group_size must be positive")
    if w.stride(-1) != 1 or w.data_ptr() % 4:
        w = w.contiguous()
    G = (K + group_size - 1) // group_size
    dev = w.device
    cols = K // 2 if qt == _lib.QUANT_INT4 else K
    packed = torch.empty((N, cols), dtype=torch.uint8 if qt == _lib.QUANT_INT4 else torch.int8, device=dev)
    scales = torch.empty((N, G), dtype=torch.float16, device=dev)
    zeros = torch.empty((N, G), dtype=torch.float16, device=dev)
    if N == 0 or K == 0:
        return packed, scales, zeros
    with torch.cuda.device(dev):
        rc = _L.mq_quantize(_ptr(w), w.stride(0), _ptr(packed), cols, _ptr(scales), _ptr(zeros), N, K,
                            group_size, qt, _stream_handle(dev))
    _check(rc)
    return packed, scales, zeros


# ---------------------------------------------------------------------------
# matmul (the fp16 vecmat route) and fast.swiglu
# ---------------------------------------------------------------------------

def _vecmat_route(M: int, N: int, K: int, dtype: torch.dtype) -> bool:
    """select_kernel's VecMat condition (src/ops/matmul.mm:177-178), for the
    dtypes this build has a kernel for."""
    return M <= 8 and N >= 256 and K >= 256 and dtype in (torch.float16, torch.float32)


def matmul(a: torch.Tensor, b: torch.Tensor, transpose_a: bool = False,
           transpose_b: bool = False) -> torch.Tensor:
    """``_C.matmul``: ``a @ op(b)``.

    The M<=8 fp16 and fp32 routes (the reference's vecmat kernels) run on this
    library's kernels; ``b`` is ``[K, N]``, or ``[N, K]`` with ``transpose_b``
    (the documented contract, include/metal_native/ops/matmul.h:18-37).
    Shapes outside that route are the reference's non-quantized
    simd32/tiled64/MPSGraph GEMMs, which this build does not re-implement:
    they are computed by torch.matmul on the GPU (hipBLASLt).
    """
    op = "matmul"
    if a.dim() < 2:
        _invalid("matmul: input 'a' must have at least 2 dimensions")
    if b.dim() < 2:
        _invalid("matmul: input 'b' must have at least 2 dimensions")
    if a.dtype != b.dtype:
        _invalid("matmul: input dtypes must match")
    _require_cuda(a, "a", op)
    _require_cuda(b, "b", op)
    M = a.shape[-1] if transpose_a else a.shape[-2]
    Ka = a.shape[-2] if transpose_a else a.shape[-1]
    Kb = b.shape[-1] if transpose_b else b.shape[-2]
    N = b.shape[-2] if transpose_b else b.shape[-1]
    if Ka != Kb:
        _invalid("matmul: incompatible dimensions for matrix multiplication")
    K = Ka
    if transpose_a or b.dim() != 2 or not _vecmat_route(M, N, K, a.dtype):
        aa = a.transpose(-1, -2) if transpose_a else a
        bb = b.transpose(-1, -2) if transpose_b else b
        return torch.matmul(aa, bb)
    lead = a.shape[:-2]
    a2 = a.reshape(-1, K)
    if a2.stride(-1) != 1:
        a2 = a2.contiguous()
    if b.stride(-1) != 1:
        b = b.contiguous()
    b, ldb = _rowmajor(b, "b", op)
    rows = a2.shape[0]
    out = torch.empty((rows, N), dtype=a.dtype, device=a.device)
    dev = a.device
    fn = _L.mq_vecmat_f16 if a.dtype == torch.float16 else _L.mq_vecmat_f32
    with torch.cuda.device(dev):
        for r0 in range(0, rows, 64):
            r1 = min(rows, r0 + 64)
            ai, lda = _rowmajor(a2[r0:r1], "a", op)
            rc = fn(_ptr(ai), lda, _ptr(b), ldb, _ptr(out[r0:r1]), N, r1 - r0, N, K, 1 if transpose_b else 0,
                    _stream_handle(dev))
            _check(rc)
    return out.reshape(*lead, M, N)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``fast.swiglu``: ``half(silu(float(gate)) * float(up))``
    (src/future/future_stubs.mm:61-101, shaders/fused_swiglu.metal:48-84)."""
    op = "fast::swiglu"
    _require_cuda(gate, "gate", op)
    _require_cuda(up, "up", op)
    if gate.dtype != up.dtype:
        _invalid("fast::swiglu: gate and up must have same dtype")
    if gate.numel() != up.numel():
        _invalid("fast::swiglu: gate and up must have same number of elements")
    if gate.dtype != torch.float16:
        _invalid("fast::swiglu: this build implements Float16")
    g = gate.contiguous()
    u = up.contiguous()
    out = torch.empty_like(g)
    dev = g.device
    with torch.cuda.device(dev):
        rc = _L.mq_swiglu_f16(_ptr(g), _ptr(u), _ptr(out), g.numel(), _stream_handle(dev))
    _check(rc)
    return out


# ---------------------------------------------------------------------------
# decoder glue (extension: the synthetic decode step of BASELINE config 5)
# ---------------------------------------------------------------------------

def add_rmsnorm(x: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``x += delta`` (fp16, in place; skipped when ``delta`` is None), then
    returns ``half(x * rsqrt(mean(x^2) + eps) * weight)`` per row."""
    for t, what in ((x, "x"), (weight, "weight")):
        _require_cuda(t, what, "add_rmsnorm")
    if x.dtype != torch.float16 or not x.is_contiguous():
        _invalid("add_rmsnorm: x must be contiguous Float16")
    n = x.shape[-1]
    rows = x.numel() // n
    out = torch.empty_like(x)
    _check(_L.mq_add_rmsnorm_f16(_ptr(x), _ptr(delta), _ptr(weight), _ptr(out), rows, n, float(eps),
                                 _stream_handle(x.device)))
    return out


def rope_kv(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor,
            v_cache: torch.Tensor, heads: int, kv_heads: int, head_dim: int) -> torch.Tensor:
    """Rotary embedding of q and k from a fused qkv row; writes k and v into
    the caches ``[kv_heads, max_len, head_dim]`` at device position ``pos``;
    returns rotated q ``[heads, head_dim]``."""
    q = torch.empty((heads, head_dim), dtype=torch.float16, device=qkv.device)
    _check(_L.mq_rope_kv_f16(_ptr(qkv), _ptr(cos), _ptr(sin), _ptr(pos), _ptr(q), _ptr(k_cache), _ptr(v_cache),
                             heads, kv_heads, head_dim, k_cache.shape[1], _stream_handle(qkv.device)))
    return q


def attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                     scale: float) -> torch.Tensor:
    """One-token grouped-query attention over cache positions ``<= pos``;
    returns fp16 ``[1, heads * head_dim]``."""
    heads, head_dim = q.shape
    L = k_cache.shape[1]
    out = torch.empty((1, heads * head_dim), dtype=torch.float16, device=q.device)
    wsb = _L.mq_attention_decode_workspace_size(heads, head_dim, L)
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=q.device)
    _check(_L.mq_attention_decode_f16(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(pos), _ptr(out), heads,
                                      k_cache.shape[0], head_dim, L, float(scale), _ptr(ws), wsb,
                                      _stream_handle(q.device)))
    return out


def rmsnorm_dequant_matmul(x: torch.Tensor, delta: torch.Tensor | None, norm_weight: torch.Tensor, eps: float,
                           resid_out: torch.Tensor, weights_packed: torch.Tensor, scales: torch.Tensor,
                           zeros: torch.Tensor | None, group_size: int, quant_type: str, epilogue: str | None = None,
                           bias: torch.Tensor | None = None) -> torch.Tensor:
    """Decode step glue fused into the GEMV (one row): ``resid_out =
    half(x + delta)``, ``h = half(resid_out * rsqrt(mean(resid_out^2) + eps) *
    norm_weight)``, returns ``dequant_matmul(h, ...)``.  One launch where the
    row-block kernel takes the shape, else ``add_rmsnorm`` + ``dequant_matmul``."""
    qt = quant_type_code(quant_type)
    epi = _EPILOGUES[epilogue]
    N, cols = weights_packed.shape
    K = x.shape[-1]
    if (x.numel() == K and resid_out is not x and resid_out is not delta
            and _L.mq_rmsnorm_dequant_matmul_supported(N, K, group_size, qt, epi)):
        n_out = N // 2 if epi == _lib.EPILOGUE_SWIGLU else N
        out = torch.empty((1, n_out), dtype=torch.float16, device=x.device)
        weights_packed, ldw = _rowmajor(weights_packed, "weights_packed", "dequant_matmul")
        rc = _L.mq_rmsnorm_dequant_matmul(_ptr(x), _ptr(delta), _ptr(norm_weight), float(eps), _ptr(resid_out),
                                          _ptr(weights_packed), ldw,
                                          _ptr(scales), _ptr(zeros), _ptr(out), N, K, group_size, qt, epi, _ptr(bias),
                                          _stream_handle(x.device))
        if rc == 0:
            return out
        if rc != 4:
            _check(rc)
    resid_out.copy_(x)
    h = add_rmsnorm(resid_out, delta, norm_weight, eps)
    return dequant_matmul(h.reshape(-1, K), weights_packed, scales, zeros, group_size, quant_type, epilogue=epilogue,
                          bias=bias)


def attention_decode_rope_supported(heads: int, head_dim: int, max_len: int) -> bool:
    """Whether ``attention_decode_rope`` runs the one-launch kernel for this shape."""
    return bool(_L.mq_attention_decode_rope_supported(heads, head_dim, max_len))


def attention_decode_rope(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor,
                          k_cache: torch.Tensor, v_cache: torch.Tensor, heads: int, kv_heads: int, head_dim: int,
                          scale: float) -> torch.Tensor:
    """``rope_kv`` followed by ``attention_decode``: one launch where
    ``attention_decode_rope_supported``, else the two separate kernels."""
    if not attention_decode_rope_supported(heads, head_dim, k_cache.shape[1]):
        q = rope_kv(qkv, cos, sin, pos, k_cache, v_cache, heads, kv_heads, head_dim)
        return attention_decode(q, k_cache, v_cache, pos, scale)
    out = torch.empty((1, heads * head_dim), dtype=torch.float16, device=qkv.device)
    _check(_L.mq_attention_decode_rope_f16(_ptr(qkv), _ptr(cos), _ptr(sin), _ptr(pos), _ptr(k_cache), _ptr(v_cache),
                                           _ptr(out), heads, kv_heads, head_dim, k_cache.shape[1], float(scale),
                                           _stream_handle(qkv.device)))
    return out


def argmax_embed_workspace(vocab: int, device) -> torch.Tensor:
    """Zeroed workspace for ``argmax_embed``; keep one per stream."""
    nb = _L.mq_argmax_embed_workspace_size(int(vocab))
    if nb < 0:
        raise MetalNativeError(f"argmax_embed: vocabulary size {vocab} not supported")
    return torch.zeros(nb, dtype=torch.uint8, device=device)


def argmax_embed(logits: torch.Tensor, embed: torch.Tensor, token: torch.Tensor, pos: torch.Tensor,
                 x: torch.Tensor, workspace: torch.Tensor) -> None:
    """Greedy decode tail in one launch, in place: ``token[0] =
    argmax(logits)`` (torch.argmax order: NaN above every number, ties to
    the lowest index), ``pos[0] += 1`` and ``x[0] = embed[token]``."""
    V = logits.numel()
    d = embed.shape[1]
    if logits.dtype != torch.float16 or embed.dtype != torch.float16 or x.dtype != torch.float16:
        raise MetalNativeError("argmax_embed: logits, embed and x must be Float16")
    if token.dtype != torch.int64 or pos.dtype != torch.int64 or token.numel() < 1 or pos.numel() < 1:
        raise MetalNativeError("argmax_embed: token and pos must be Int64 with one element")
    if not logits.is_contiguous() or embed.stride(1) != 1 or not x.is_contiguous() or x.numel() < d:
        raise MetalNativeError("argmax_embed: contiguous logits and x, embed rows with unit stride")
    if embed.shape[0] != V:
        raise MetalNativeError("argmax_embed: embed must have one row per logit")
    for t in (logits, embed, token, pos, x, workspace):
        if t.device != logits.device or t.device.type != "cuda":
            raise MetalNativeError("argmax_embed: all tensors must be on the same GPU")
    _check(_L.mq_argmax_embed_f16(_ptr(logits), V, _ptr(embed), embed.stride(0), d, _ptr(token), _ptr(pos), _ptr(x),
                                  _ptr(workspace), workspace.numel(), _stream_handle(logits.device)))


def synchronize() -> None:
    """``_C.synchronize``: wait for all queued GPU work."""
    torch.cuda.synchronize()


def set_option(key: str, value: int) -> None:
    """Kernel-path override for tests/tuning (see mq_set_option)."""
    _check(_L.mq_set_option(key.encode(), int(value)))


def last_path() -> str:
    return _lib.PATH_NAMES.get(_L.mq_last_path(), "unknown")
