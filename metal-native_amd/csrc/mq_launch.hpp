// Internal launcher interface between the C-ABI (mq_capi.cpp) and the kernel
// translation units.  Host-only declarations; no torch types anywhere.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mq {

enum Fmt { FMT_INT4 = 0, FMT_INT8 = 1, FMT_F16 = 2 };
enum Epi { EPI_NONE = 0, EPI_BIAS = 1, EPI_SWIGLU = 2 };

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

// Persistent row-range GEMV (decode, M <= 16).
struct DecodeTuning {
  int rpw = 0;           // weight rows per MFMA tile (0 = from M and K)
  int max_nw = 16;       // wavefronts per workgroup
  int wg_per_cu = 1;     // workgroups per CU the rows are spread over
  int force_chunks = 0;  // tests: stage K in at least this many chunks
};
struct DecodePlan {
  int rpw, nw, rows_wg, nwg, nsteps, spc, nchunks, xs_stride, xp;
  uint32_t off_szs, off_red, off_bnd, off_ws;
  int sz_chunks;
  size_t lds_bytes;
  bool ok;
};
bool decode_supported(const LinearArgs& a);
DecodePlan decode_plan(const LinearArgs& a, int num_cus, const DecodeTuning& t);
hipError_t decode_launch(const LinearArgs& a, const DecodePlan& p, hipStream_t s);

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
