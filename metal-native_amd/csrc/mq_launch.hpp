// Internal launcher interface between the C-ABI (mq_capi.cpp) and the kernel
// translation units.  Host-only declarations; no torch types anywhere.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mq {

enum Fmt { FMT_INT4 = 0, FMT_INT8 = 1, FMT_F16 = 2 };
enum Epi { EPI_NONE = 0, EPI_BIAS = 1, EPI_SWIGLU = 2 };

// Split-K workspace layout: a fixed-size counter region (zero between calls)
// followed by the fp32 partial sums.  The counter region's size does not
// depend on the problem, so partials of one call never overlap counters of
// another call that shares the workspace.
constexpr size_t kWsCounterBytes = 65536;

// One quantized (or fp16) linear: C[M, Nout] = epi(A[M,K] . W[N,K]^T).
struct LinearArgs {
  const void* A;        // fp16 [M, K], row stride lda (elements)
  int64_t lda;
  const void* W;        // int4 [N, K/2] u8, int8 [N, K], or fp16 [N, K] (row stride ldw elements of W's type)
  int64_t ldw;          // row stride of W in bytes
  const void* scales;   // fp16 [N, G] (unused for fp16 W)
  const void* zeros;    // fp16 [N, G] or nullptr (= no zero term)
  const void* bias;     // fp16 [N] for EPI_BIAS
  void* C;              // fp16 [M, Nout], row stride ldc (elements)
  int64_t ldc;
  int M, N, K;
  int g, G;             // group size along K, groups per row
  int fmt;              // Fmt
  int epi;              // Epi
  int F;                // SwiGLU half width (N = 2F), 0 otherwise
};

// Split-K launch geometry chosen on the host for the skinny kernel.
struct SkinnyPlan {
  int steps;      // 16-byte loads per lane per K chunk
  int mblocks;    // 16-row blocks of A (M <= 16*mblocks)
  int splits;     // number of K chunks (grid.y)
  int kchunk;     // K elements per chunk
  int rblocks;    // weight-row blocks (grid.x)
  size_t lds_bytes;
  size_t ws_bytes;  // workspace needed (counters + partials); 0 if splits == 1
  int nofence;      // timing experiments only
};

bool skinny_supported(const LinearArgs& a);
SkinnyPlan skinny_plan(const LinearArgs& a, int num_cus, size_t ws_avail);
hipError_t skinny_launch(const LinearArgs& a, const SkinnyPlan& p, void* ws, hipStream_t s);

// Row-block GEMV (no split-K workspace).
struct GemvTuning {
  bool allow_full = true;  // whole-K activations in LDS when they fit
  int max_nw = 16;         // cap on wavefronts per workgroup
  int rpw = 0;             // weight rows per unit (0 = by M)
};
struct GemvPlan {
  int nw;         // wavefronts per workgroup (K split inside the workgroup)
  int rpw;        // weight rows per unit (whole-K kernel)
  int xs_stride;  // LDS activation row stride in halves (whole-K kernel)
  int mblocks;    // 16-row blocks of A
  int rowblocks;  // workgroups (16 weight rows each)
  int nchunks;    // K chunks (one step per wave each)
  int nsteps;     // K steps of 4 16-byte pieces per row
  int kpad;       // K rounded up to whole steps
  bool xfull;     // whole activation matrix staged in LDS
  size_t lds_bytes;
};
bool gemv_supported(const LinearArgs& a);
GemvPlan gemv_plan(const LinearArgs& a, const GemvTuning& t);
hipError_t gemv_launch(const LinearArgs& a, const GemvPlan& p, hipStream_t s);

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

hipError_t swiglu_launch(const void* gate, const void* up, void* out, int64_t n, hipStream_t s);

// fp16 GEMV with B stored [K, N] (transpose_b == false): C = A . B.
hipError_t vecmat_kn_launch(const void* A, int64_t lda, const void* B, int64_t ldb,
                            void* C, int64_t ldc, int M, int N, int K, hipStream_t s);

}  // namespace mq
