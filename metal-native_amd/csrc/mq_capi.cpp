// C-ABI entry points: argument validation (mirroring src/ops/matmul.mm:910-934),
// kernel-path selection and launch.  The caller owns inputs and outputs; the
// split-K GEMV's partial sums and counters live in a library workspace, one
// per (device, stream), allocated and zeroed on first use and grown on demand.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "../../include/metal_native_amd.h"
#include "mq_launch.hpp"

namespace {

thread_local std::string g_last_error;
thread_local int g_last_path = 0;
std::atomic<int> g_force_path{0};
std::atomic<int> g_gemv_steps{0};
std::atomic<int> g_gemv_tpw{0};

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return e == hipErrorOutOfMemory ? MQ_OUT_OF_MEMORY : MQ_INTERNAL_ERROR;
}

int num_cus_current() {
  static std::atomic<int> cache[64] = {};   // per device; threads may race to fill in the same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Path ids (mq_last_path / force_path); 1 and 5 are retired ids of earlier
// decode kernels and are not reused.
// PATH_TILED selects the prefill GEMM family (force_path); the kernel that ran
// is reported as PATH_GEMM16 (the 16x16x32 register-dequant GEMM), PATH_GEMMW
// (register-operand 32x32x16 GEMM), PATH_GEMMW_SPLIT (the same with K split
// over workgroups) or PATH_TILED (the 16x16x32 fallback).
enum Path {
  PATH_AUTO = 0, PATH_TILED = 2, PATH_GENERIC = 3, PATH_VECMAT_KN = 4, PATH_DECODE = 6, PATH_ROWS = 7,
  PATH_GEMMW = 8, PATH_VECMAT32 = 9, PATH_GEMMW_SPLIT = 10, PATH_GEMM16 = 11, PATH_RSTREAM = 12
};
// prefill GEMM choice (gemm_impl): 0 automatic (the register-dequant GEMM where
// its tiles fill the GPU, else the register-operand 32x32x16 kernel where it
// takes the shape), 1 always the 16x16x32 tiled kernel, 2 the register-dequant
// GEMM wherever it takes the shape
std::atomic<int> g_gemm_impl{0};
// gemm_split: 1 lets the 32x32x16 kernel split K over workgroups where its
// tiles leave CUs idle, 0 keeps one workgroup per tile
std::atomic<int> g_gemm_split{1};

mq::GemvTuning gemv_tuning() {
  mq::GemvTuning t;
  t.steps = g_gemv_steps.load();
  t.tpw = g_gemv_tpw.load();
  return t;
}

bool decode_ok(const mq::LinearArgs& a) {
  return mq::gemv_supported(a) && mq::gemv_plan(a, num_cus_current(), gemv_tuning()).ok;
}

// Split-K workspace, one per (device, stream): counters must start at zero and
// every launch leaves them at zero, so one fill at allocation suffices.
// Calls on one stream are ordered, so they may share it.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
std::vector<void*> g_ws_retired;   // superseded workspaces: kept until the process ends

hipError_t workspace_for(hipStream_t s, size_t need, void** out) {
  *out = nullptr;
  if (need == 0) return hipSuccess;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  Workspace& w = g_ws[{dev, s}];
  if (w.bytes < need) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return hipErrorStreamCaptureUnsupported;  // first call on this stream must be outside capture
    size_t nb = need < ((size_t)1 << 20) ? ((size_t)1 << 20) : need;
    // A superseded buffer is kept, not freed: graphs captured earlier on
    // this stream hold its address and may still be replayed.  Growth is
    // geometric, so the retired buffers add up to less than the live one.
    if (nb < 2 * w.bytes) nb = 2 * w.bytes;
    void* p = nullptr;
    e = hipMalloc(&p, nb);
    if (e != hipSuccess) return e;
    // zeroed on the stream that uses it, so the first kernel on that stream
    // is ordered after the fill whatever the stream's flags (never inside a
    // capture: refused above)
    e = hipMemsetAsync(p, 0, nb, s);
    if (e != hipSuccess) { (void)hipFree(p); return e; }
    if (w.ptr) g_ws_retired.push_back(w.ptr);
    w.ptr = p;
    w.bytes = nb;
  }
  *out = w.ptr;
  return hipSuccess;
}

bool rows_ok(const mq::LinearArgs& a) { return mq::rows_plan(a, num_cus_current()).ok; }

bool prefill_ok(const mq::LinearArgs& a) {
  return mq::gemm16_supported(a) || mq::gemmw_supported(a, num_cus_current()) || mq::tiled_supported(a);
}

// The 16x16x32 GEMM (mq_gemm16.hip), automatically: where its tiles cover
// the CUs at least three quarters of the way and its row blocks (128 rows;
// 64 for int8 SwiGLU up to M = 64) are at least three quarters full
// (config 3, M = 512: 256 tiles on 256 CUs; config 4, M = 64: 237 tiles).
// Smaller grids go to the 32x32x16 kernel, whose planner picks narrower
// tiles or splits K.
bool gemm16_auto(const mq::LinearArgs& a) {
  if (!mq::gemm16_supported(a)) return false;
  const int bm = mq::gemm16_rows_per_tile(a);
  const int64_t mpad = (int64_t)((a.M + bm - 1) / bm) * bm;
  return 4 * (int64_t)mq::gemm16_workgroups(a) >= 3 * (int64_t)num_cus_current() && 4 * (int64_t)a.M >= 3 * mpad;
}

// Short weight rows over many of them, M <= 4: the split-K GEMV, whose
// start-up is shorter than the row-block kernel's staging of all of K.
// Measured on 108 shapes (M = 1, 2, 4; K = 512..3584; N = 896, 4864, 14336;
// int4 g64 and int8 per-channel): it is faster for K <= 896 from N = 4864
// (config 1, K = 896, N = 4864: 4.0 vs 5.2 us) and for int4 at K = 1536
// with M <= 2 (4.6 vs 5.6 us at N = 4864), slower at N = 896 and from K = 2048.
bool short_rows(const mq::LinearArgs& a) {
  if (a.prenorm || a.fmt == mq::FMT_F16) return false;
  const int64_t nrows = a.epi == mq::EPI_SWIGLU ? a.F : a.N;
  if (nrows < 2048) return false;
  return a.K <= 1024 || (a.fmt == mq::FMT_INT4 && a.M <= 2 && a.K <= 1536);
}

int choose_path(const mq::LinearArgs& a, bool noalloc) {
  int forced = g_force_path.load();
  if (forced == PATH_ROWS && rows_ok(a)) return PATH_ROWS;
  if (forced == PATH_RSTREAM && mq::rstream_plan(a, num_cus_current()).ok) return PATH_RSTREAM;
  if (forced == PATH_DECODE && decode_ok(a)) return PATH_DECODE;
  if (forced == PATH_TILED && prefill_ok(a)) return PATH_TILED;
  if (forced == PATH_GENERIC) return PATH_GENERIC;
  // automatic choice: the row-block kernel up to M = 4; for M = 5..16 only
  // where the activations fit in LDS whole (its K parts measured slower than
  // the split-K GEMV at config 2, M = 8: 20.3 vs 18.2 us; whole, it is
  // faster: config 4 at M = 8, 29.5 vs 40.3 us, at M = 16, 31.8 vs 45.4 us)
  if (a.M <= 4 && short_rows(a) && decode_ok(a)) return PATH_DECODE;
  if (a.M <= 4 && rows_ok(a)) return PATH_ROWS;
  if (a.M <= 16) {
    const mq::RowsPlan pl = mq::rows_plan(a, num_cus_current());
    if (pl.ok && pl.KP == 1) return PATH_ROWS;
  }
  // M = 5..16 whose activations do not fit in LDS whole: the register-streamed
  // GEMV where its plan takes the shape (no K parts, no workspace; config 2 at
  // M = 5 / 8: 15.0 / 16.1 us against 17.0 / 18.5 us for the row-block
  // kernel's K parts and 17.6 us for the split-K GEMV at M = 8; at M = 9..16
  // 6-45 % faster than both the K-split prefill GEMM and the split-K GEMV
  // on 13 shapes, e.g. config 2 at M = 9 / 16: 19.0-19.7 / 21.6 us against
  // 25.0 / 25.4 us, K = 4096, N = 4096, M = 16: 8.3 against 12.0 us)
  if (a.M >= 5 && a.M <= 16 && mq::rstream_plan(a, num_cus_current()).ok) return PATH_RSTREAM;
  // M = 9..16 with long rows the register-streamed plan declines: the prefill GEMM with K split over
  // workgroups beats the split-K GEMV (measured at K >= 8192 on 6 shapes at
  // M = 9, 12, 13-16: faster on all but K = 8192, N = 4096 (2-10 % slower
  // at M = 9-16), by up to 45 %, e.g. K = 18944, N = 3584, M = 16: 26.3 vs
  // 40.0 us; at K = 4096, N = 4096 it is 8 % slower, hence the K bound)
  if (a.M >= 9 && a.K >= 8192 && !noalloc && g_gemm_impl.load() == 0 && g_gemm_split.load() != 0 &&
      mq::gemmw_supported(a, num_cus_current()) && mq::gemmw_ws_bytes(a, num_cus_current(), true) > 0)
    return PATH_TILED;
  if (decode_ok(a)) return PATH_DECODE;
  if (prefill_ok(a)) return PATH_TILED;
  return PATH_GENERIC;
}

// noalloc: the split-K GEMV uses the library's fixed scratch array instead of
// the per-stream workspace (no allocation on any path).
int run_linear(const mq::LinearArgs& a, hipStream_t s, bool noalloc = false) {
  int path = choose_path(a, noalloc);
  hipError_t e = hipSuccess;
  if (path == PATH_ROWS) {
    // K parts need the workspace: the no-allocation entry point takes the
    // split-K GEMV (whose scratch is fixed) for such shapes
    const mq::RowsPlan pl = mq::rows_plan(a, num_cus_current(), !noalloc);
    if (pl.ok) {
      void* ws = nullptr;
      e = workspace_for(s, pl.ws_bytes, &ws);
      if (e == hipErrorStreamCaptureUnsupported)
        return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: the split-K workspace of this stream is too small; "
                                         "make one call of this shape on the stream before capturing it");
      if (e != hipSuccess) return hip_fail(e, "dequant_matmul: workspace allocation failed");
      e = mq::rows_launch(a, pl, ws, s);
    } else {
      path = decode_ok(a) ? PATH_DECODE : PATH_GENERIC;
    }
  }
  if (path == PATH_RSTREAM) {
    const mq::RsPlan pl = mq::rstream_plan(a, num_cus_current());
    e = pl.ok ? mq::rstream_launch(a, pl, s) : hipErrorInvalidValue;
  } else if (path == PATH_ROWS) {
  } else if (path == PATH_DECODE) {
    const mq::GemvPlan pl = mq::gemv_plan(a, num_cus_current(), gemv_tuning());
    void* ws = nullptr;
    if (noalloc) {
      if (pl.ws_bytes > mq::gemv_scratch_bytes())
        return fail(MQ_INVALID_ARGUMENT, "dequant_matmul_noalloc: the split-K partial sums of this shape need " +
                                             std::to_string(pl.ws_bytes) + " bytes, more than the fixed scratch of " +
                                             std::to_string(mq::gemv_scratch_bytes()) + " bytes");
      if (pl.ws_bytes) {
        e = mq::gemv_scratch(s, &ws);
        if (e != hipSuccess) return hip_fail(e, "dequant_matmul_noalloc: scratch set-up failed");
      }
    } else {
      e = workspace_for(s, pl.ws_bytes, &ws);
      if (e == hipErrorStreamCaptureUnsupported && a.M <= 4 && rows_ok(a)) {
        // under capture with a workspace too small for this shape: the
        // row-block kernel in one part (no workspace) rather than an error
        const mq::RowsPlan rp = mq::rows_plan(a, num_cus_current(), false);
        if (rp.ok) {
          path = PATH_ROWS;
          e = mq::rows_launch(a, rp, nullptr, s);
          if (e != hipSuccess) return hip_fail(e, "dequant_matmul: kernel launch failed");
          g_last_path = path;
          return MQ_SUCCESS;
        }
      }
      if (e == hipErrorStreamCaptureUnsupported)
        return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: the split-K workspace of this stream is too small; "
                                         "make one call of this shape on the stream before capturing it");
      if (e != hipSuccess) return hip_fail(e, "dequant_matmul: workspace allocation failed");
    }
    e = mq::gemv_launch(a, pl, ws, s);
  } else if (path == PATH_TILED) {
    const int impl = g_gemm_impl.load();
    // K split over workgroups needs the per-stream workspace: the
    // no-allocation entry point keeps one workgroup per tile
    auto gemmw = [&]() -> hipError_t {
      const int cus = num_cus_current();
      bool split = !noalloc && g_gemm_split.load() != 0;
      void* ws = nullptr;
      size_t need = split ? mq::gemmw_ws_bytes(a, cus, true) : 0;
      hipError_t we = workspace_for(s, need, &ws);
      if (we == hipErrorStreamCaptureUnsupported) {
        // under capture with a workspace too small for this shape: one
        // workgroup per tile (no workspace) rather than an error
        split = false;
        need = 0;
        ws = nullptr;
        we = hipSuccess;
      }
      if (we != hipSuccess) return we;
      path = need ? PATH_GEMMW_SPLIT : PATH_GEMMW;
      return mq::gemmw_launch(a, cus, ws, s, split);
    };
    if ((impl == 0 && gemm16_auto(a)) || (impl == 2 && mq::gemm16_supported(a))) {
      e = mq::gemm16_launch(a, s, nullptr);
      path = PATH_GEMM16;
    } else if ((impl == 0 || impl == 2) && mq::gemmw_supported(a, num_cus_current())) {
      e = gemmw();
    } else if (mq::tiled_supported(a)) {
      e = mq::tiled_launch(a, s);
    } else if (mq::gemmw_supported(a, num_cus_current())) {
      e = gemmw();
    } else {
      e = mq::generic_linear_launch(a, s);
      path = PATH_GENERIC;
    }
  } else {
    e = mq::generic_linear_launch(a, s);
  }
  if (e == hipErrorStreamCaptureUnsupported)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: the split-K workspace of this stream is too small; "
                                     "make one call of this shape on the stream before capturing it");
  if (e != hipSuccess) return hip_fail(e, "dequant_matmul: kernel launch failed");
  g_last_path = path;
  return MQ_SUCCESS;
}

// Validation shared by the linear entry points.
int build_args(mq::LinearArgs& a, int64_t M, int64_t N, int64_t K, int32_t group_size,
               int32_t quant_type, int32_t epilogue) {
  if (M < 1 || N < 1 || K < 1)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: M, N and K must be positive");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: dimension too large");
  if (group_size < 1)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: group_size must be positive");
  if (quant_type != MQ_QUANT_INT4 && quant_type != MQ_QUANT_INT8)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: quant_type must be INT4 or INT8");
  if (quant_type == MQ_QUANT_INT4 && (K & 1))
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: INT4 weights must be [N, K/2] with K even");
  if (epilogue < MQ_EPILOGUE_NONE || epilogue > MQ_EPILOGUE_SWIGLU)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: unknown epilogue");
  static_assert(MQ_EPILOGUE_BIAS == mq::EPI_BIAS && MQ_EPILOGUE_BIAS_RELU == mq::EPI_BIAS_RELU &&
                    MQ_EPILOGUE_BIAS_SILU == mq::EPI_BIAS_SILU && MQ_EPILOGUE_RESIDUAL == mq::EPI_RESIDUAL &&
                    MQ_EPILOGUE_SWIGLU == mq::EPI_SWIGLU,
                "C ABI and kernel epilogue numbering agree");
  if (epilogue == MQ_EPILOGUE_SWIGLU && (N & 1))
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: SwiGLU needs an even number of weight rows");
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.g = group_size;
  a.G = (int)((K + group_size - 1) / group_size);
  a.fmt = quant_type == MQ_QUANT_INT4 ? mq::FMT_INT4 : mq::FMT_INT8;
  a.epi = epilogue;
  a.F = epilogue == MQ_EPILOGUE_SWIGLU ? (int)(N / 2) : 0;
  return MQ_SUCCESS;
}

}  // namespace

namespace mq {

hipError_t allow_dynamic_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(mu);
  if (done.count({kernel, dev})) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert({kernel, dev});
  return e;
}

}  // namespace mq

extern "C" {

static int dequant_matmul_impl(bool noalloc, const void* activations, int64_t lda, const void* weights_packed,
                             int64_t ldw_bytes, const void* scales, const void* zeros, void* out,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size,
                             int32_t quant_type, int32_t epilogue, const void* bias, const void* residual,
                             int64_t ldr, void* stream) {
  mq::LinearArgs a{};
  int rc = build_args(a, M, N, K, group_size, quant_type, epilogue);
  if (rc != MQ_SUCCESS) return rc;
  if (!activations || !weights_packed || !scales || !out)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: null pointer argument");
  if (mq::epi_needs_bias(epilogue) && !bias)
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: bias epilogue needs a bias pointer");
  if (epilogue == MQ_EPILOGUE_RESIDUAL) {
    if (!residual) return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: residual epilogue needs a residual pointer");
    if (ldr < N) return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: ldr must be >= N");
    if (residual == out && ldr != ldc)
      return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: a residual that is the output needs ldr == ldc");
  }
  const int64_t row_bytes = quant_type == MQ_QUANT_INT4 ? K / 2 : K;
  if (lda < K) return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: lda must be >= K");
  if (ldw_bytes < row_bytes)
    return fail(MQ_INVALID_ARGUMENT, quant_type == MQ_QUANT_INT4
                                         ? "dequant_matmul: INT4 weights must be [N, K/2]"
                                         : "dequant_matmul: INT8 weights must be [N, K]");
  if (ldc < (epilogue == MQ_EPILOGUE_SWIGLU ? N / 2 : N))
    return fail(MQ_INVALID_ARGUMENT, "dequant_matmul: ldc too small");
  a.A = activations; a.lda = lda;
  a.W = weights_packed; a.ldw = ldw_bytes;
  a.scales = scales; a.zeros = zeros; a.bias = bias;
  a.resid = residual; a.ldr = ldr;
  a.C = out; a.ldc = ldc;
  return run_linear(a, (hipStream_t)stream, noalloc);
}

MQ_API int mq_dequant_matmul(const void* activations, int64_t lda, const void* weights_packed,
                             int64_t ldw_bytes, const void* scales, const void* zeros, void* out,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size,
                             int32_t quant_type, int32_t epilogue, const void* bias, const void* residual,
                             int64_t ldr, void* stream) {
  return dequant_matmul_impl(false, activations, lda, weights_packed, ldw_bytes, scales, zeros, out, ldc, M, N, K,
                             group_size, quant_type, epilogue, bias, residual, ldr, stream);
}

MQ_API int mq_dequant_matmul_noalloc(const void* activations, int64_t lda, const void* weights_packed,
                                     int64_t ldw_bytes, const void* scales, const void* zeros, void* out,
                                     int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size,
                                     int32_t quant_type, int32_t epilogue, const void* bias, const void* residual,
                                     int64_t ldr, void* stream) {
  return dequant_matmul_impl(true, activations, lda, weights_packed, ldw_bytes, scales, zeros, out, ldc, M, N, K,
                             group_size, quant_type, epilogue, bias, residual, ldr, stream);
}

MQ_API int mq_rmsnorm_dequant_matmul(const void* x, const void* delta, const void* norm_weight, float eps,
                                     void* resid_out, const void* weights_packed, int64_t ldw_bytes,
                                     const void* scales, const void* zeros, void* C, int64_t N, int64_t K,
                                     int32_t group_size, int32_t quant_type, int32_t epilogue, const void* bias,
                                     void* stream) {
  if (!x || !norm_weight || !resid_out)
    return fail(MQ_INVALID_ARGUMENT, "rmsnorm_dequant_matmul: null pointer argument");
  if (resid_out == x || (delta && resid_out == delta))
    return fail(MQ_INVALID_ARGUMENT, "rmsnorm_dequant_matmul: resid_out must not alias x or delta");
  mq::LinearArgs a{};
  int rc = build_args(a, 1, N, K, group_size, quant_type, epilogue);
  if (rc != MQ_SUCCESS) return rc;
  a.A = x; a.lda = K;
  a.W = weights_packed; a.ldw = ldw_bytes;
  a.scales = scales; a.zeros = zeros; a.bias = bias;
  a.C = C; a.ldc = a.epi == mq::EPI_SWIGLU ? a.F : N;
  a.prenorm = 1; a.pre_delta = delta; a.pre_weight = norm_weight; a.pre_resid = resid_out; a.pre_eps = eps;
  if (!weights_packed || !scales || !C) return fail(MQ_INVALID_ARGUMENT, "rmsnorm_dequant_matmul: null pointer argument");
  if (mq::epi_needs_bias(epilogue) && !bias)
    return fail(MQ_INVALID_ARGUMENT, "rmsnorm_dequant_matmul: bias epilogue needs a bias pointer");
  if (epilogue == MQ_EPILOGUE_RESIDUAL)
    return fail(MQ_INVALID_ARGUMENT, "rmsnorm_dequant_matmul: the residual epilogue is not fused here");
  if (ldw_bytes < (quant_type == MQ_QUANT_INT4 ? K / 2 : K))
    return fail(MQ_INVALID_ARGUMENT, "rmsnorm_dequant_matmul: weight rows too short");
  const mq::RowsPlan pl = mq::rows_plan(a, num_cus_current());
  if (!pl.ok) return fail(MQ_INVALID_ARGUMENT, "rmsnorm_dequant_matmul: shape not supported by the fused kernel");
  hipError_t e = mq::rows_launch(a, pl, nullptr, (hipStream_t)stream);   // pre-norm: one K part, no workspace
  if (e != hipSuccess) return hip_fail(e, "rmsnorm_dequant_matmul: kernel launch failed");
  g_last_path = PATH_ROWS;
  return MQ_SUCCESS;
}

MQ_API int mq_rmsnorm_dequant_matmul_supported(int64_t N, int64_t K, int32_t group_size, int32_t quant_type,
                                               int32_t epilogue) {
  mq::LinearArgs a{};
  if (build_args(a, 1, N, K, group_size, quant_type, epilogue) != MQ_SUCCESS) return 0;
  static const uint64_t kAligned[2] = {0, 0};  // stand-in pointers: only the shape is asked about
  a.A = a.W = a.scales = kAligned;
  a.lda = K;
  a.ldw = quant_type == MQ_QUANT_INT4 ? K / 2 : K;
  a.prenorm = 1; a.pre_weight = a.pre_resid = (void*)kAligned;
  return mq::rows_plan(a, num_cus_current()).ok ? 1 : 0;
}

MQ_API int mq_dequantize(const void* weights_packed, int64_t ldw_bytes, const void* scales,
                         const void* zeros, void* out, int64_t ldo, int64_t N, int64_t K,
                         int32_t group_size, int32_t quant_type, int32_t flat_groups, void* stream) {
  if (!weights_packed || !scales || !out) return fail(MQ_INVALID_ARGUMENT, "dequantize: null pointer argument");
  if (N < 1 || K < 1 || N * K > ((int64_t)1 << 40)) return fail(MQ_INVALID_ARGUMENT, "dequantize: bad shape");
  if (group_size < 1) return fail(MQ_INVALID_ARGUMENT, "dequantize: group_size must be positive");
  if (quant_type != MQ_QUANT_INT4 && quant_type != MQ_QUANT_INT8)
    return fail(MQ_INVALID_ARGUMENT, "dequantize: quant_type must be INT4 or INT8");
  if (flat_groups && zeros) return fail(MQ_INVALID_ARGUMENT, "dequantize: flat groups take no zeros");
  if (!flat_groups && quant_type == MQ_QUANT_INT4 && (K & 1))
    return fail(MQ_INVALID_ARGUMENT, "dequantize: INT4 rows need an even K");
  if (ldo < K) return fail(MQ_INVALID_ARGUMENT, "dequantize: ldo must be >= K");
  if (!flat_groups && ldw_bytes < (quant_type == MQ_QUANT_INT4 ? K / 2 : K))
    return fail(MQ_INVALID_ARGUMENT, "dequantize: weight rows too short");
  mq::DequantArgs a{};
  a.W = weights_packed; a.ldw = ldw_bytes;
  a.scales = scales; a.zeros = zeros;
  a.out = out; a.ldo = ldo;
  a.N = (int)N; a.K = (int)K; a.g = group_size;
  a.G = (int)((K + group_size - 1) / group_size);
  a.fmt = quant_type == MQ_QUANT_INT4 ? mq::FMT_INT4 : mq::FMT_INT8;
  a.flat = flat_groups ? 1 : 0;
  if (a.flat) {  // flat layout is one contiguous element range
    a.ldw = quant_type == MQ_QUANT_INT4 ? K / 2 : K;
    if (a.ldo != K) return fail(MQ_INVALID_ARGUMENT, "dequantize: flat groups need ldo == K");
  }
  hipError_t e = mq::dequantize_launch(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dequantize: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int mq_quantize(const void* w, int64_t ldw, void* weights_packed, int64_t ldo_bytes, void* scales,
                       void* zeros, int64_t N, int64_t K, int32_t group_size, int32_t quant_type, void* stream) {
  if (!w || !weights_packed || !scales || !zeros) return fail(MQ_INVALID_ARGUMENT, "quantize: null pointer argument");
  if (N < 1 || K < 1 || N > INT32_MAX || K > INT32_MAX) return fail(MQ_INVALID_ARGUMENT, "quantize: bad shape");
  if (group_size < 1) return fail(MQ_INVALID_ARGUMENT, "quantize: group_size must be positive");
  if (quant_type != MQ_QUANT_INT4 && quant_type != MQ_QUANT_INT8)
    return fail(MQ_INVALID_ARGUMENT, "quantize: quant_type must be INT4 or INT8");
  if (quant_type == MQ_QUANT_INT4 && ((K & 1) || (group_size & 1)))
    return fail(MQ_INVALID_ARGUMENT, "quantize: INT4 needs an even K and an even group_size");
  if (ldw < K) return fail(MQ_INVALID_ARGUMENT, "quantize: ldw must be >= K");
  if (ldo_bytes < (quant_type == MQ_QUANT_INT4 ? K / 2 : K))
    return fail(MQ_INVALID_ARGUMENT, "quantize: output rows too short");
  if ((uintptr_t)w & 3) return fail(MQ_INVALID_ARGUMENT, "quantize: weights must be 4-byte aligned");
  mq::QuantizeArgs a{};
  a.W = w; a.ldw = ldw; a.out = weights_packed; a.ldo = ldo_bytes;
  a.scales = scales; a.zeros = zeros;
  a.N = (int)N; a.K = (int)K; a.g = group_size;
  a.G = (int)((K + group_size - 1) / group_size);
  a.fmt = quant_type == MQ_QUANT_INT4 ? mq::FMT_INT4 : mq::FMT_INT8;
  hipError_t e = mq::quantize_launch(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "quantize: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int mq_vecmat_f16(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc,
                         int64_t M, int64_t N, int64_t K, int32_t transpose_b, void* stream) {
  if (!a || !b || !c) return fail(MQ_INVALID_ARGUMENT, "matmul: null pointer argument");
  if (M < 1 || N < 1 || K < 1 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MQ_INVALID_ARGUMENT, "matmul: bad shape");
  if (lda < K || ldc < N || ldb < (transpose_b ? K : N))
    return fail(MQ_INVALID_ARGUMENT, "matmul: leading dimension too small");
  if (!transpose_b) {
    hipError_t e = mq::vecmat_kn_launch(a, lda, b, ldb, c, ldc, (int)M, (int)N, (int)K, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "matmul: kernel launch failed");
    g_last_path = PATH_VECMAT_KN;
    return MQ_SUCCESS;
  }
  mq::LinearArgs la{};
  la.A = a; la.lda = lda;
  la.W = b; la.ldw = ldb * 2;
  la.C = c; la.ldc = ldc;
  la.M = (int)M; la.N = (int)N; la.K = (int)K;
  la.g = 1; la.G = 1;
  la.fmt = mq::FMT_F16;
  la.epi = mq::EPI_NONE;
  const int pth = choose_path(la, false);
  if (pth == PATH_DECODE || pth == PATH_ROWS) return run_linear(la, (hipStream_t)stream);
  hipError_t e = mq::generic_linear_launch(la, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "matmul: kernel launch failed");
  g_last_path = PATH_GENERIC;
  return MQ_SUCCESS;
}

MQ_API int mq_vecmat_f32(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc,
                         int64_t M, int64_t N, int64_t K, int32_t transpose_b, void* stream) {
  if (!a || !b || !c) return fail(MQ_INVALID_ARGUMENT, "matmul: null pointer argument");
  if (M < 1 || N < 1 || K < 1 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MQ_INVALID_ARGUMENT, "matmul: bad shape");
  if (lda < K || ldc < N || ldb < (transpose_b ? K : N))
    return fail(MQ_INVALID_ARGUMENT, "matmul: leading dimension too small");
  hipError_t e = mq::vecmat32_launch(a, lda, b, ldb, c, ldc, (int)M, (int)N, (int)K, transpose_b != 0,
                                     (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "matmul: kernel launch failed");
  g_last_path = PATH_VECMAT32;
  return MQ_SUCCESS;
}

MQ_API int mq_swiglu_f16(const void* gate, const void* up, void* out, int64_t n, void* stream) {
  if (!gate || !up || !out) return fail(MQ_INVALID_ARGUMENT, "fast::swiglu: null pointer argument");
  if (n < 0) return fail(MQ_INVALID_ARGUMENT, "fast::swiglu: negative size");
  if (n == 0) return MQ_SUCCESS;
  hipError_t e = mq::swiglu_launch(gate, up, out, n, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "fast::swiglu: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int mq_add_rmsnorm_f16(void* x, const void* delta, const void* weight, void* out, int64_t rows, int64_t n,
                              float eps, void* stream) {
  if (!x || !weight || !out) return fail(MQ_INVALID_ARGUMENT, "add_rmsnorm: null pointer argument");
  if (rows < 1 || n < 1 || rows > INT32_MAX || n > INT32_MAX) return fail(MQ_INVALID_ARGUMENT, "add_rmsnorm: bad shape");
  hipError_t e = mq::add_rmsnorm_launch(x, delta, weight, out, (int)rows, (int)n, eps, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "add_rmsnorm: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int mq_rope_kv_f16(const void* qkv, const float* cos_table, const float* sin_table, const int64_t* pos,
                          void* q_out, void* k_cache, void* v_cache, int32_t heads, int32_t kv_heads,
                          int32_t head_dim, int64_t max_len, void* stream) {
  if (!qkv || !cos_table || !sin_table || !pos || !q_out || !k_cache || !v_cache)
    return fail(MQ_INVALID_ARGUMENT, "rope_kv: null pointer argument");
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 2 || (head_dim & 1) || max_len < 1)
    return fail(MQ_INVALID_ARGUMENT, "rope_kv: bad shape");
  hipError_t e = mq::rope_kv_launch(qkv, cos_table, sin_table, pos, q_out, k_cache, v_cache, heads, kv_heads,
                                    head_dim, max_len, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "rope_kv: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int64_t mq_attention_decode_workspace_size(int32_t heads, int32_t head_dim, int64_t max_len) {
  if (heads < 1 || head_dim < 1 || max_len < 1) return -1;
  return (int64_t)mq::attn_decode_workspace(heads, head_dim, max_len);
}

MQ_API int mq_attention_decode_f16(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos,
                                   void* out, int32_t heads, int32_t kv_heads, int32_t head_dim, int64_t max_len,
                                   float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !pos || !out || !workspace)
    return fail(MQ_INVALID_ARGUMENT, "attention_decode: null pointer argument");
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 8 || head_dim > 512 || (head_dim & 7) ||
      max_len < 1)
    return fail(MQ_INVALID_ARGUMENT, "attention_decode: bad shape");
  if (workspace_bytes < (int64_t)mq::attn_decode_workspace(heads, head_dim, max_len))
    return fail(MQ_INVALID_ARGUMENT, "attention_decode: workspace too small");
  hipError_t e = mq::attn_decode_launch(q, k_cache, v_cache, pos, out, heads, kv_heads, head_dim, max_len, scale,
                                        workspace, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "attention_decode: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int mq_attention_decode_rope_supported(int32_t heads, int32_t head_dim, int64_t max_len) {
  return heads >= 1 && max_len >= 1 && mq::attn_fused_supported(heads, head_dim, max_len) ? 1 : 0;
}

MQ_API int mq_attention_decode_rope_f16(const void* qkv, const float* cos_table, const float* sin_table,
                                        const int64_t* pos, void* k_cache, void* v_cache, void* out, int32_t heads,
                                        int32_t kv_heads, int32_t head_dim, int64_t max_len, float scale,
                                        void* stream) {
  if (!qkv || !cos_table || !sin_table || !pos || !k_cache || !v_cache || !out)
    return fail(MQ_INVALID_ARGUMENT, "attention_decode_rope: null pointer argument");
  if (heads < 1 || kv_heads < 1 || heads % kv_heads || max_len < 1 ||
      !mq::attn_fused_supported(heads, head_dim, max_len))
    return fail(MQ_INVALID_ARGUMENT, "attention_decode_rope: bad shape (head_dim 64 or 128, max_len <= 4096)");
  hipError_t e = mq::attn_fused_launch(qkv, cos_table, sin_table, pos, k_cache, v_cache, out, heads, kv_heads,
                                       head_dim, max_len, scale, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "attention_decode_rope: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int64_t mq_argmax_embed_workspace_size(int64_t vocab) {
  if (vocab < 1 || vocab > (int64_t)INT32_MAX - 2048) return -1;
  return (int64_t)mq::argmax_embed_workspace(vocab);
}

MQ_API int mq_argmax_embed_f16(const void* logits, int64_t vocab, const void* embed, int64_t embed_stride, int64_t d,
                               int64_t* token, int64_t* pos, void* x, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  if (!logits || !embed || !token || !pos || !x || !workspace)
    return fail(MQ_INVALID_ARGUMENT, "argmax_embed: null pointer argument");
  if (vocab < 1 || vocab > (int64_t)INT32_MAX - 2048 || d < 1 || d > INT32_MAX || embed_stride < d)
    return fail(MQ_INVALID_ARGUMENT, "argmax_embed: bad shape");
  if (workspace_bytes < (int64_t)mq::argmax_embed_workspace(vocab))
    return fail(MQ_INVALID_ARGUMENT, "argmax_embed: workspace too small");
  hipError_t e = mq::argmax_embed_launch(logits, vocab, embed, embed_stride, (int)d, token, pos, x, workspace,
                                         (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "argmax_embed: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int64_t mq_read_probe_sink_size(void) { return (int64_t)12 * num_cus_current() * 4; }

MQ_API int mq_read_probe(const void* p, int64_t bytes, void* sink, void* stream) {
  if (!p || !sink) return fail(MQ_INVALID_ARGUMENT, "read_probe: null pointer argument");
  if (bytes < 1 || bytes >= ((int64_t)1 << 31)) return fail(MQ_INVALID_ARGUMENT, "read_probe: bytes must be in [1, 2^31)");
  hipError_t e = mq::read_probe_launch(p, bytes, sink, num_cus_current(), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "read_probe: kernel launch failed");
  return MQ_SUCCESS;
}

MQ_API int mq_set_option(const char* key, int64_t value) {
  if (!key) return fail(MQ_INVALID_ARGUMENT, "set_option: null key");
  if (std::strcmp(key, "force_path") == 0) {
    if (value != PATH_AUTO && value != PATH_TILED && value != PATH_GENERIC && value != PATH_DECODE &&
        value != PATH_ROWS && value != PATH_RSTREAM)
      return fail(MQ_INVALID_ARGUMENT, "set_option: force_path must be 0, 2, 3, 6, 7 or 12");
    g_force_path.store((int)value);
    return MQ_SUCCESS;
  }
  if (std::strcmp(key, "gemm_impl") == 0) {
    if (value != 0 && value != 1 && value != 2)
      return fail(MQ_INVALID_ARGUMENT, "set_option: gemm_impl must be 0, 1 or 2");
    g_gemm_impl.store((int)value);
    return MQ_SUCCESS;
  }
  if (std::strcmp(key, "gemm_split") == 0) {
    if (value != 0 && value != 1) return fail(MQ_INVALID_ARGUMENT, "set_option: gemm_split must be 0 or 1");
    g_gemm_split.store((int)value);
    return MQ_SUCCESS;
  }
  if (std::strcmp(key, "gemv_steps") == 0) {
    if (value < 0 || value > 8) return fail(MQ_INVALID_ARGUMENT, "set_option: gemv_steps must be 0..8");
    g_gemv_steps.store((int)value);
    return MQ_SUCCESS;
  }
  if (std::strcmp(key, "gemv_tiles_per_wg") == 0) {
    if (value != 0 && value != 1 && value != 2 && value != 4)
      return fail(MQ_INVALID_ARGUMENT, "set_option: gemv_tiles_per_wg must be 0, 1, 2 or 4");
    g_gemv_tpw.store((int)value);
    return MQ_SUCCESS;
  }
  return fail(MQ_INVALID_ARGUMENT, std::string("set_option: unknown key ") + key);
}

MQ_API int mq_last_path(void) { return g_last_path; }

MQ_API const char* mq_last_error(void) { return g_last_error.c_str(); }

MQ_API const char* mq_error_to_string(int code) {
  switch (code) {
    case MQ_SUCCESS: return "Success";
    case MQ_DEVICE_NOT_FOUND: return "DeviceNotFound";
    case MQ_ALLOCATION_FAILED: return "AllocationFailed";
    case MQ_KERNEL_COMPILATION_FAILED: return "KernelCompilationFailed";
    case MQ_INVALID_ARGUMENT: return "InvalidArgument";
    case MQ_OUT_OF_MEMORY: return "OutOfMemory";
    case MQ_TIMEOUT_ERROR: return "TimeoutError";
    case MQ_INTERNAL_ERROR: return "InternalError";
    case MQ_NOT_IMPLEMENTED: return "NotImplemented";
    default: return "Unknown";
  }
}

MQ_API int mq_abi_version(void) { return 3; }

}  // extern "C"
