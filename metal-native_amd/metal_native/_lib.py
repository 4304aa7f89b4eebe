"""ctypes binding of libmetal_native_amd.so (the C ABI in include/metal_native_amd.h).

torch is imported before the library is loaded so that the HIP runtime torch
ships is the one the library binds to (one runtime per process; torch's
stream handles are then valid arguments).  There is no fallback: if the
library is missing, importing this module raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded first, see module docstring)

LIB_NAME = "libmetal_native_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# status codes: include/metal_native/core/error.h:21-31 numbering
SUCCESS = 0
INVALID_ARGUMENT = 4

QUANT_INT4 = 0
QUANT_INT8 = 1

# include/metal_native/ops/fused_matmul.h:18-24 numbering, plus SwiGLU
EPILOGUE_NONE = 0
EPILOGUE_BIAS = 1
EPILOGUE_BIAS_RELU = 2
EPILOGUE_BIAS_SILU = 3
EPILOGUE_RESIDUAL = 4
EPILOGUE_SWIGLU = 5

PATH_NAMES = {0: "none", 2: "tiled", 3: "generic", 4: "vecmat_kn", 6: "decode", 7: "rows", 8: "gemmw", 9: "vecmat_f32", 10: "gemmw_split",
              11: "gemm16", 12: "rstream"}

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> (restype, argtypes)
SIGNATURES = {
    "mq_read_probe_sink_size": (_i64, []),
    "mq_read_probe": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p]),
    "mq_dequant_matmul": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
                                 _i64, _i64, _i64, _i64, _i32, _i32, _i32, _c_void_p, _c_void_p, _i64,
                                 _c_void_p]),
    "mq_dequant_matmul_noalloc": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
                                         _i64, _i64, _i64, _i64, _i32, _i32, _i32, _c_void_p, _c_void_p, _i64,
                                         _c_void_p]),
    "mq_dequantize": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                             _i32, _i32, _i32, _c_void_p]),
    "mq_rmsnorm_dequant_matmul": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.c_float, _c_void_p, _c_void_p,
                                         _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32, _i32,
                                         _c_void_p, _c_void_p]),
    "mq_rmsnorm_dequant_matmul_supported": (_i32, [_i64, _i64, _i32, _i32, _i32]),
    "mq_quantize": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32,
                           _c_void_p]),
    "mq_vecmat_f16": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _i64,
                             _i32, _c_void_p]),
    "mq_vecmat_f32": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _i64,
                             _i32, _c_void_p]),
    "mq_swiglu_f16": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "mq_add_rmsnorm_f16": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, ctypes.c_float,
                                  _c_void_p]),
    "mq_rope_kv_f16": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                              _i32, _i32, _i32, _i64, _c_void_p]),
    "mq_attention_decode_workspace_size": (_i64, [_i32, _i32, _i64]),
    "mq_attention_decode_rope_supported": (_i32, [_i32, _i32, _i64]),
    "mq_attention_decode_rope_f16": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                            _c_void_p, _i32, _i32, _i32, _i64, ctypes.c_float, _c_void_p]),
    "mq_attention_decode_f16": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32,
                                       _i64, ctypes.c_float, _c_void_p, _i64, _c_void_p]),
    "mq_argmax_embed_workspace_size": (_i64, [_i64]),
    "mq_argmax_embed_f16": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                   _c_void_p, _i64, _c_void_p]),
    "mq_set_option": (_i32, [ctypes.c_char_p, _i64]),
    "mq_last_path": (_i32, []),
    "mq_last_error": (ctypes.c_char_p, []),
    "mq_error_to_string": (ctypes.c_char_p, [_i32]),
    "mq_abi_version": (_i32, []),
}


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is not built; run `python metal-native_amd/build.py` "
            "(or __graft_entry__.build()) first")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()
