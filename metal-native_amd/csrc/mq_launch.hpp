// Internal launcher interface between the C-ABI (mq_capi.cpp) and the kernel
// translation units.  Host-only declarations; no torch types anywhere.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mq {

enum Fmt { FMT_INT4 = 0, FMT_INT8 = 1, FMT_F16 = 2 };
// Epilogues, numbered like the reference's MatmulEpilogue
// (include/metal_native/ops/fused_matmul.h:18-24), plus SwiGLU.  The first
// five are element-wise on the fp32 accumulator (EpiArgs below); SwiGLU pairs
// two weight rows per output and changes a kernel's shape, so kernels take it
// as a template parameter and the element-wise ones as a run-time value.
enum Epi { EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_RELU = 2, EPI_BIAS_SILU = 3, EPI_RESIDUAL = 4, EPI_SWIGLU = 5 };
__host__ __device__ inline bool epi_needs_bias(int e) { return e == EPI_BIAS || e == EPI_BIAS_RELU || e == EPI_BIAS_SILU; }

// Operands of the element-wise epilogues: bias fp16 [N], residual fp16
// [M, N] with row stride ldr elements (it may be the output itself when
// ldr == ldc: every output element is read and written by one thread).
struct EpiArgs {
  const void* bias;
  const void* resid;
  int64_t ldr;
  int epi;
};

// One quantized (or fp16) linear: C[M, Nout] = epi(A[M,K] . W[N,K]^T).
struct LinearArgs {
  const void* A;        // fp16 [M, K], row stride lda (elements)
  int64_t lda;
  const void* W;        // int4 [N, K/2] u8, int8 [N, K], or fp16 [N, K] (row stride ldw elements of W's type)
  int64_t ldw;          // row stride of W in bytes
  const void* scales;   // fp16 [N, G] (unused for fp16 W)
  const void* zeros;    // fp16 [N, G] or nullptr (= no zero term)
  const void* bias;     // fp16 [N] for the bias epilogues
  const void* resid;    // fp16 [M, N] (row stride ldr) for EPI_RESIDUAL
  int64_t ldr;
  void* C;              // fp16 [M, Nout], row stride ldc (elements)
  int64_t ldc;
  int M, N, K;
  int g, G;             // group size along K, groups per row
  int fmt;              // Fmt
  int epi;              // Epi
  __host__ __device__ EpiArgs epi_args() const { return EpiArgs{bias, resid, ldr, epi}; }
  int F;                // SwiGLU half width (N = 2F), 0 otherwise
  // Optional fused pre-norm (row-block GEMV, M = 1): the activations are
  // A' = half(A + pre_delta) (pre_delta may be null), written to pre_resid by
  // one workgroup, then RMS-normalised: half(A' * rsqrt(mean(A'^2) + eps) * w).
  int prenorm = 0;
  const void* pre_delta = nullptr;
  const void* pre_weight = nullptr;
  void* pre_resid = nullptr;
  float pre_eps = 0.f;
};

// Raise a kernel's dynamic LDS limit to `bytes` on the current device, once
// per (kernel, device); thread-safe.
hipError_t allow_dynamic_lds(const void* kernel, int bytes);

// Split-K MFMA GEMV (decode, M <= 16).
struct GemvTuning {
  int steps = 0;   // K steps per wave, 1..8 (0 = planner's choice)
  int tpw = 0;     // row tiles (= waves) per workgroup: 1, 2 or 4 (0 = planner's choice)
};
struct GemvPlan {
  int rpw, tpw, P, kk, nq, nwg, KS, T, GK, XS;
  uint32_t off_sz;
  size_t lds_bytes;
  size_t cnt_bytes;  // counter region at the start of the workspace
  size_t ws_bytes;   // 0 when P == 1
  bool ok;
};
bool gemv_supported(const LinearArgs& a);
GemvPlan gemv_plan(const LinearArgs& a, int num_cus, const GemvTuning& t);
// ws: ws_bytes of device memory whose first cnt_bytes are zero (the kernel
// leaves them zero again); calls sharing a workspace must be stream-ordered.
hipError_t gemv_launch(const LinearArgs& a, const GemvPlan& p, void* ws, hipStream_t s);
// Fixed split-K scratch for callers that cannot allocate: a file-scope
// device array of gemv_scratch_bytes() bytes.  gemv_scratch returns its
// address on the current device; the first call on a device looks the
// symbol up and clears its counters with a kernel on stream s.
size_t gemv_scratch_bytes();
hipError_t gemv_scratch(hipStream_t s, void** ptr);

// Persistent row-block GEMV (decode with the activations resident in LDS).
// KP > 1 splits K into parts (activations too long for LDS); the parts of a
// row block meet through ws_bytes of the per-stream workspace.
struct RowsPlan {
  int rpw, mh, nw, nwg, R, TW, KS, XS, maxT, snp;   // mh: activation-row halves (2: M = 9..16 on 8-row tiles)
  int KP, nblk, KStot;
  uint32_t off_sz, off_scr, off_slot, off_wft;
  size_t lds_bytes, ws_bytes;
  bool ok;
};
RowsPlan rows_plan(const LinearArgs& a, int num_cus, bool allow_split = true);
hipError_t rows_launch(const LinearArgs& a, const RowsPlan& p, void* ws, hipStream_t s);

// Register-streamed row-block decode GEMV (mq_rstream.hip): int4 weights,
// 3 <= M <= 16, long K, no workspace.
struct RsPlan {
  int rpw, twm, R, TW, KS, nwg;
  bool ok;
};
RsPlan rstream_plan(const LinearArgs& a, int num_cus);
hipError_t rstream_launch(const LinearArgs& a, const RsPlan& p, hipStream_t s);

// Register-operand 32x32x16 MFMA GEMM (prefill default).  Where its tiles
// leave CUs idle it may split K over several workgroups per tile (only when
// allow_split), which needs a zeroed workspace of gemmw_ws_bytes (counters
// that every launch leaves at zero, then the partial sums).
bool gemmw_supported(const LinearArgs& a, int num_cus);
size_t gemmw_ws_bytes(const LinearArgs& a, int num_cus, bool allow_split);
hipError_t gemmw_launch(const LinearArgs& a, int num_cus, void* ws, hipStream_t s, bool allow_split);

// 128-row int4 GEMM (16x16x32 MFMA, one workgroup per 128 x 80 tile, no
// workspace).  trace: optional per-wave timestamps (null in the library).
bool gemm16_supported(const LinearArgs& a);
int gemm16_workgroups(const LinearArgs& a);
int gemm16_rows_per_tile(const LinearArgs& a);
hipError_t gemm16_launch(const LinearArgs& a, hipStream_t s, uint64_t* trace);

// 16x16x32 MFMA GEMM, K steps of 32 (fallback for shapes the GEMM above does not take).
bool tiled_supported(const LinearArgs& a);
hipError_t tiled_launch(const LinearArgs& a, hipStream_t s);

hipError_t generic_linear_launch(const LinearArgs& a, hipStream_t s);

// Dequantize weights to fp16 [N, K] (row stride ldo elements).
// flat != 0 selects the standalone-kernel semantics: group index i/g over the
// flattened element index i and no zero term.
struct DequantArgs {
  const void* W; int64_t ldw;
  const void* scales; const void* zeros;
  void* out; int64_t ldo;
  int N, K, g, G, fmt, flat;
};
hipError_t dequantize_launch(const DequantArgs& a, hipStream_t s);

// Group quantizer (the inverse of the dequant formula): W fp16 [N, K] (row
// stride ldw elements) -> out int4 [N, K/2] / int8 [N, K] (row stride ldo
// bytes), scales and zeros fp16 [N, G] contiguous.
// Division of 32-bit indices below 2^31 by a fixed d >= 1 as a multiply and a
// shift: q = (i + umulhi(i, mp)) >> l with l = ceil(log2 d) and mp =
// ceil(2^(32+l) / d) - 2^32.  Exact for every i < 2^31: the multiplier's
// excess over 2^(32+l) / d adds less than i / 2^(32+l) < 1 / (2 d) to i / d.
struct Div32 {
  uint32_t mp;
  int l;
  static Div32 make(uint32_t d) {
    int l = 0;
    while ((1ull << l) < d) ++l;
    const unsigned __int128 m = ((((unsigned __int128)1) << (32 + l)) + d - 1) / d;
    return {(uint32_t)(m - ((unsigned __int128)1 << 32)), l};
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t i) const {
    return (i + (uint32_t)(((uint64_t)i * mp) >> 32)) >> l;
  }
};

struct QuantizeArgs {
  const void* W; int64_t ldw;
  void* out; int64_t ldo;
  void* scales; void* zeros;
  int N, K, g, G, fmt;
};
hipError_t quantize_launch(const QuantizeArgs& a, hipStream_t s);

// Decoder glue (synthetic decode step).
hipError_t add_rmsnorm_launch(void* x, const void* delta, const void* w, void* out, int rows, int n, float eps,
                              hipStream_t s);
hipError_t rope_kv_launch(const void* qkv, const float* cos_t, const float* sin_t, const int64_t* pos, void* q_out,
                          void* kc, void* vc, int H, int KVH, int D, int64_t L, hipStream_t s);
size_t attn_decode_workspace(int H, int D, int64_t L);
// rotary + cache write + attention in one launch, one workgroup per query head
// (head_dim 64 or 128, L <= 4096)
bool attn_fused_supported(int H, int D, int64_t L);
hipError_t attn_fused_launch(const void* qkv, const float* cos_t, const float* sin_t, const int64_t* pos, void* kc,
                             void* vc, void* out, int H, int KVH, int D, int64_t L, float scale, hipStream_t s);
hipError_t attn_decode_launch(const void* q, const void* kc, const void* vc, const int64_t* pos, void* out, int H,
                              int KVH, int D, int64_t L, float scale, void* ws, hipStream_t s);

// greedy decode tail: tok = argmax(logits[V]) (torch.argmax order), pos += 1,
// x[d] = embed row tok (row stride lde); ws: argmax_embed_workspace bytes whose
// leading counter is zero (every launch leaves it zero)
size_t argmax_embed_workspace(int64_t V);
hipError_t argmax_embed_launch(const void* logits, int64_t V, const void* embed, int64_t lde, int d, int64_t* tok,
                               int64_t* pos, void* x, void* ws, hipStream_t s);

hipError_t swiglu_launch(const void* gate, const void* up, void* out, int64_t n, hipStream_t s);
// One-launch read of `bytes` bytes (measurement aid); sink: 12 * num_cus u32.
hipError_t read_probe_launch(const void* p, int64_t bytes, void* sink, int num_cus, hipStream_t s);

// fp16 GEMV with B stored [K, N] (transpose_b == false): C = A . B.
hipError_t vecmat_kn_launch(const void* A, int64_t lda, const void* B, int64_t ldb,
                            void* C, int64_t ldc, int M, int N, int K, hipStream_t s);

// fp32 GEMV, any M (launches of 8 rows): C = A . B (B [K, N]) or A . B^T (B [N, K]).
hipError_t vecmat32_launch(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int M,
                           int N, int K, bool transpose_b, hipStream_t s);

}  // namespace mq
