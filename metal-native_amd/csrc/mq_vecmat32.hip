// fp32 vector-matrix products for skinny A (M <= 8 rows per launch): the
// fp32 side of _C.matmul's vecmat route, C = A . op(B) in fp32.
//
// Replaces matmul_vecmat_fp32 and matmul_vecmat_batch_fp32
// (shaders/matmul_vecmat_kernel.metal:286-369, :462-534; selected at
// src/ops/matmul.mm:213-225 for M <= 8, N >= 256, K >= 256, :177-178), with
// the documented contract C = A . B for B [K, N] and C = A . B^T for
// B [N, K] (transpose_b), as the fp16 route of this library.
//
// Both are HBM-bound on B (read once); A is small and reused from LDS.  The
// products accumulate with fmaf (one rounding per multiply-add).
//  * B [N, K]: a workgroup of 4 waves owns 8 consecutive rows of B (2 per
//    wave).  A is staged in LDS in K-chunks of 1024; a lane reads 16 bytes of
//    each of its wave's rows per step (one coalesced 1 KiB load per row and
//    wave), takes the matching A pieces from LDS and keeps 2 x M fp32
//    partial sums; a wave reduction gives each output.
//  * B [K, N]: a workgroup of 8 waves owns 64 consecutive columns; a lane
//    holds 4 columns of one of 32 row slots, so one wave load reads 4 rows x
//    256 contiguous bytes (16-byte pieces: the texture unit's fast pattern);
//    the partial sums meet by shuffles and in LDS in a fixed order
//    (deterministic).  A is staged in LDS in K-chunks (one broadcast LDS read
//    per multiply).  Unaligned operands take a scalar variant (one column
//    per lane, 16 waves).
#include "mq_device.hpp"
#include "mq_launch.hpp"

namespace mq {
namespace {

constexpr int kChunk = 1024;   // k per staged A chunk ([N, K] kernel)
constexpr int kRows = 2;       // B rows per wave ([N, K] kernel)
constexpr int kWavesKN = 16;   // waves per workgroup ([K, N] kernel)
constexpr int kChunkKN = 512;  // k per staged A chunk ([K, N] kernel)

// Loads below are unconditional, at an index clamped into the operand, and
// the value is replaced by zero afterwards where it lies outside (a select:
// whatever the clamped element holds, NaN included, is discarded).  Loads
// under a branch would each be waited for before the next is issued.
//
// Stage A[0..M)[k0 .. k0 + kc) into as (zeros past kc): every thread's loads
// are issued before any of its LDS stores, so the chunk costs one memory
// round trip, not one per element.
template <int M, int CH, int NT>
__device__ __forceinline__ void stage_a(float (&as)[M][CH], const float* A, int64_t lda, int k0, int kc, int tid) {
  constexpr int PER = (M * CH + NT - 1) / NT;
  float t[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int i = tid + e * NT, m = i / CH, k = i - m * CH;
    const float v = A[(int64_t)min(m, M - 1) * lda + k0 + min(k, kc - 1)];
    t[e] = (i < M * CH && k < kc) ? v : 0.f;
  }
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int i = tid + e * NT, m = i / CH, k = i - m * CH;
    if (i < M * CH) as[m][k] = t[e];
  }
}

template <int M>
__global__ __launch_bounds__(256) void vecmat32_nk_kernel(const float* A, int64_t lda, const float* B, int64_t ldb,
                                                          float* C, int64_t ldc, int N, int K, int vec) {
  __shared__ __align__(16) float as[M][kChunk];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n0 = blockIdx.x * 4 * kRows + w * kRows;   // this wave's first row
  float acc[kRows][M];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  constexpr int NIT = kChunk / 256;   // 16-byte pieces per lane and row in a chunk
  for (int k0 = 0; k0 < K; k0 += kChunk) {
    const int kc = min(kChunk, K - k0);
    // the chunk's B pieces are issued first: their latency overlaps the A staging
    float4 b[NIT][kRows];
    if (vec) {
#pragma unroll
      for (int it = 0; it < NIT; ++it)
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
          const int k = 4 * lane + 256 * it;
          const float4 v = *(const float4*)(B + (int64_t)min(n0 + r, N - 1) * ldb + k0 + (k < kc ? k : 0));
          b[it][r] = (n0 + r < N && k < kc) ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    __syncthreads();   // the previous chunk is consumed
    stage_a<M, kChunk, 256>(as, A, lda, k0, kc, tid);
    __syncthreads();
    if (vec) {   // rows 16-byte aligned, K a multiple of 4 (pieces past the chunk are zero)
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int k = 4 * lane + 256 * it;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float4 a = *(const float4*)&as[m][k];
#pragma unroll
          for (int r = 0; r < kRows; ++r)
            acc[r][m] = fmaf(a.w, b[it][r].w, fmaf(a.z, b[it][r].z, fmaf(a.y, b[it][r].y, fmaf(a.x, b[it][r].x, acc[r][m]))));
        }
      }
    } else {
      for (int k = lane; k < kc; k += 64) {
        float b[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
          const float v = B[(int64_t)min(n0 + r, N - 1) * ldb + k0 + k];
          b[r] = n0 + r < N ? v : 0.f;
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float a = as[m][k];
#pragma unroll
          for (int r = 0; r < kRows; ++r) acc[r][m] = fmaf(a, b[r], acc[r][m]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v = acc[r][m];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += xor_lane(v, o);
      if (lane == 0 && n0 + r < N) C[(int64_t)m * ldc + n0 + r] = v;
    }
}

template <int M>
__global__ __launch_bounds__(64 * kWavesKN) void vecmat32_kn_kernel(const float* A, int64_t lda, const float* B,
                                                                    int64_t ldb, float* C, int64_t ldc, int N, int K) {
  __shared__ float as[M][kChunkKN];
  __shared__ float red[kWavesKN][M][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = blockIdx.x * 64 + lane;
  const bool on = n < N;
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;
  constexpr int NR = kChunkKN / kWavesKN;   // rows of B per wave and chunk
  for (int k0 = 0; k0 < K; k0 += kChunkKN) {
    const int kc = min(kChunkKN, K - k0);
    // wave w takes rows k = w, w + 16, ... of the chunk; all of them are
    // issued before the A staging, so their latency overlaps it
    float b[NR];
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const int k = w + u * kWavesKN;
      const float v = B[(int64_t)(k0 + min(k, kc - 1)) * ldb + min(n, N - 1)];
      b[u] = (on && k < kc) ? v : 0.f;
    }
    __syncthreads();   // the previous chunk is consumed
    stage_a<M, kChunkKN, 64 * kWavesKN>(as, A, lda, k0, kc, tid);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NR; ++u)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[m] = fmaf(as[m][w + u * kWavesKN], b[u], acc[m]);   // zero past the chunk
  }
#pragma unroll
  for (int m = 0; m < M; ++m) red[w][m][lane] = acc[m];
  __syncthreads();
  if (w < M && on) {   // wave m sums output row m over the waves, in wave order
    float sum = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWavesKN; ++ww) sum += red[ww][w][lane];
    C[(int64_t)w * ldc + n] = sum;
  }
}

// B [K, N] with 16-byte rows pieces (ldb % 4 == 0, N % 4 == 0, B 16-byte
// aligned): 8 waves on 64 columns; lane (g, c) holds columns 4c..4c+3 and row
// slot 4w + g, so one wave load reads four rows x 256 contiguous bytes.  The
// partial sums meet across the row groups by shuffles and across the waves
// in LDS, in a fixed order.
constexpr int kWavesKV = 8;
template <int M>
__global__ __launch_bounds__(64 * kWavesKV) void vecmat32_kn4_kernel(const float* A, int64_t lda, const float* B,
                                                                     int64_t ldb, float* C, int64_t ldc, int N, int K) {
  constexpr int NS = 4 * kWavesKV;            // row slots per workgroup
  constexpr int NRL = kChunkKN / NS;          // rows per lane and chunk
  __shared__ float as[M][kChunkKN];
  __shared__ float4 red[kWavesKV][M][16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int cg = lane & 15, slot = 4 * w + (lane >> 4);
  const int n = blockIdx.x * 64 + 4 * cg;
  const bool on = n < N;
  const int nc = on ? n : N - 4;   // a real column group for the discarded loads
  float4 acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < K; k0 += kChunkKN) {
    const int kc = min(kChunkKN, K - k0);
    float4 b[NRL];
#pragma unroll
    for (int u = 0; u < NRL; ++u) {
      const int k = slot + u * NS;
      const float4 v = *(const float4*)(B + (int64_t)(k0 + min(k, kc - 1)) * ldb + nc);
      b[u] = (on && k < kc) ? v : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();   // the previous chunk is consumed
    stage_a<M, kChunkKN, 64 * kWavesKV>(as, A, lda, k0, kc, tid);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NRL; ++u)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float a = as[m][slot + u * NS];   // zero past the chunk
        acc[m].x = fmaf(a, b[u].x, acc[m].x);
        acc[m].y = fmaf(a, b[u].y, acc[m].y);
        acc[m].z = fmaf(a, b[u].z, acc[m].z);
        acc[m].w = fmaf(a, b[u].w, acc[m].w);
      }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
      acc[m].x += xor_lane(acc[m].x, o);
      acc[m].y += xor_lane(acc[m].y, o);
      acc[m].z += xor_lane(acc[m].z, o);
      acc[m].w += xor_lane(acc[m].w, o);
    }
    if (lane < 16) red[w][m][cg] = acc[m];
  }
  __syncthreads();
  if (tid < M * 16) {   // thread (m, c) sums its column group over the waves, in wave order
    const int m = tid >> 4, c = tid & 15;
    const int nn = blockIdx.x * 64 + 4 * c;
    if (nn < N) {
      float4 sum = red[0][m][c];
#pragma unroll
      for (int ww = 1; ww < kWavesKV; ++ww) {
        const float4 v = red[ww][m][c];
        sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
      }
      float* cp = C + (int64_t)m * ldc + nn;
      cp[0] = sum.x; cp[1] = sum.y; cp[2] = sum.z; cp[3] = sum.w;
    }
  }
}

template <int M>
hipError_t launch_m(const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc, int N, int K,
                    bool transpose_b, hipStream_t s) {
  if (transpose_b) {
    const int vec = (K % 4 == 0) && (ldb % 4 == 0) && !((uintptr_t)B & 15);
    hipLaunchKernelGGL(vecmat32_nk_kernel<M>, dim3((N + 4 * kRows - 1) / (4 * kRows)), dim3(256), 0, s, A, lda, B,
                       ldb, C, ldc, N, K, vec);
  } else if (N % 4 == 0 && ldb % 4 == 0 && !((uintptr_t)B & 15)) {
    hipLaunchKernelGGL(vecmat32_kn4_kernel<M>, dim3((N + 63) / 64), dim3(64 * kWavesKV), 0, s, A, lda, B, ldb, C,
                       ldc, N, K);
  } else {
    hipLaunchKernelGGL(vecmat32_kn_kernel<M>, dim3((N + 63) / 64), dim3(64 * kWavesKN), 0, s, A, lda, B, ldb, C, ldc,
                       N, K);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t vecmat32_launch(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int M,
                           int N, int K, bool transpose_b, hipStream_t s) {
  // rows of A in launches of up to 8
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int mc = M - m0 < 8 ? M - m0 : 8;
    const float* a = (const float*)A + (int64_t)m0 * lda;
    float* c = (float*)C + (int64_t)m0 * ldc;
    const float* b = (const float*)B;
    hipError_t e;
    switch (mc) {
      case 1: e = launch_m<1>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
      case 2: e = launch_m<2>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
      case 3: e = launch_m<3>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
      case 4: e = launch_m<4>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
      case 5: e = launch_m<5>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
      case 6: e = launch_m<6>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
      case 7: e = launch_m<7>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
      default: e = launch_m<8>(a, lda, b, ldb, c, ldc, N, K, transpose_b, s); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mq
