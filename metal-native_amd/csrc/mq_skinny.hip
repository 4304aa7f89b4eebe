// Split-K MFMA kernel for skinny activations (decode, M <= 64).
//
// Replaces the reference's M<=8 route, dequant_matmul_int{4,8}_vecmat_fp16
// (shaders/matmul_dequant_kernel.metal:229-345, :485-576, dispatched at
// src/ops/matmul.mm:946-1009), and the fp16 vecmat route for B stored [N, K]
// (shaders/matmul_vecmat_kernel.metal:32-139).  Unlike the reference kernel,
// every row of A is computed.
//
// Work decomposition (one workgroup = 4 wavefronts of 64 lanes):
//   grid.x = weight-row block (64 rows; for SwiGLU 32 gate + the matching 32
//            up rows), grid.y = K chunk (split-K).
//   Each wave owns 16 weight rows.  Lane l handles row (l & 15) and reads one
//   16-byte piece of that row per step (lane group l>>4 picks which piece),
//   so a wave step covers 16 rows x 64 contiguous bytes.  The 16 bytes are
//   dequantized in registers straight into the B operand of
//   v_mfma_f32_16x16x32_f16; activations come from LDS as the A operand
//   (rows >= M are zero).  All weight loads of a chunk are issued before the
//   activation chunk is staged, so the HBM stream starts at once.
//   Partial sums of the K chunks are combined by the last-arriving workgroup
//   of each row block (a counter per row block, reset to zero by that
//   workgroup); it sums the partials in chunk order, so results do not
//   depend on arrival order.
#include "mq_device.hpp"
#include "mq_launch.hpp"

namespace mq {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = 64;

struct SkinnyKArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros; const _Float16* bias;
  _Float16* C; int64_t ldc;
  int M, N, K, g, G, F;
  int gshift;           // log2(g) when g is a power of two, else -1
  int splits;
  int nofence;          // timing experiments only: drop the release/acquire fences
  uint32_t* counters;   // [rblocks]
  float* partials;      // [splits, M, N]
};

__device__ __forceinline__ u4 ld16(const void* p) {
  return __builtin_nontemporal_load((const u4*)p);
}
__device__ __forceinline__ u4 ld16_cached(const void* p) { return *(const u4*)p; }

template <int FMT, int STEPS, int MB, int EPI>
__global__ __launch_bounds__(kThreads) void skinny_kernel(SkinnyKArgs p) {
  constexpr int KPL = FmtTraits<FMT>::KPL;   // k per 16-byte piece
  constexpr int KSTEP = 4 * KPL;             // k per wave step
  constexpr int KC = STEPS * KSTEP;          // k per chunk
  constexpr int XS = KC + 8;                 // LDS row stride (halves), padded
  extern __shared__ __align__(16) unsigned char smem[];
  _Float16* xs = (_Float16*)smem;                              // [M][XS]
  float* tile = (float*)(smem + (size_t)p.M * XS * 2);         // [M][64]
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rb = blockIdx.x, sidx = blockIdx.y;
  const int nloc = lane & 15, grp = lane >> 4;
  const int kbase = sidx * KC;

  // weight row of this lane
  int col_in_block = 16 * w + nloc;   // 0..63 column of the block tile
  int n;
  bool row_ok;
  if (EPI == EPI_SWIGLU) {
    int j = 32 * rb + 16 * (w & 1) + nloc;
    row_ok = j < p.F;
    n = (w >= 2) ? p.F + j : j;
  } else {
    n = kRowsPerBlock * rb + col_in_block;
    row_ok = n < p.N;
  }

  // ---- issue the weight (and scale/zero) loads of the whole chunk ----
  u4 raw[STEPS];
  _Float16 sc[STEPS], zr[STEPS];
  const unsigned char* wrow = p.W + (int64_t)(row_ok ? n : 0) * p.ldw;
#pragma unroll
  for (int t = 0; t < STEPS; ++t) {
    int kk = kbase + t * KSTEP + grp * KPL;
    bool ok = row_ok && kk < p.K;
    raw[t] = (u4){0u, 0u, 0u, 0u};
    sc[t] = (_Float16)0.0f;
    zr[t] = (_Float16)0.0f;
    if (ok) {
      constexpr int BPK2 = (FMT == FMT_INT4) ? 1 : (FMT == FMT_INT8 ? 2 : 4);  // 2*bytes per k
      raw[t] = ld16(wrow + (int64_t)kk * BPK2 / 2);
      if (FMT != FMT_F16) {
        int gi = p.gshift >= 0 ? (kk >> p.gshift) : (p.G == 1 ? 0 : kk / p.g);
        sc[t] = p.scales[(int64_t)n * p.G + gi];
        if (p.zeros) zr[t] = p.zeros[(int64_t)n * p.G + gi];
      }
    }
  }

  // ---- stage the activation chunk (permuted for int4) ----
  {
    constexpr int CPR = KC / 8;  // 16-byte pieces per row
    for (int idx = tid; idx < p.M * CPR; idx += kThreads) {
      int m = idx / CPR, c = idx - m * CPR;
      int kk = kbase + 8 * c;
      u4 v = (u4){0u, 0u, 0u, 0u};
      if (kk < p.K) v = ld16_cached(p.A + (int64_t)m * p.lda + kk);
      if (FMT == FMT_INT4) v = perm8_int4(v);
      *(u4*)(xs + m * XS + 8 * c) = v;
    }
  }
  __syncthreads();

  // ---- dequantize + MFMA ----
  f4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = (f4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < STEPS; ++t) {
    h2 s2 = (h2){sc[t], sc[t]};
    h2 z2 = (h2){zr[t], zr[t]};
#pragma unroll
    for (int j = 0; j < KPL / 8; ++j) {
      h8 b;
      if (FMT == FMT_INT4) {
        uint32_t d = (j == 0) ? raw[t].x : (j == 1) ? raw[t].y : (j == 2) ? raw[t].z : raw[t].w;
        b = dq_int4_dword_perm(d, s2, z2);
      } else if (FMT == FMT_INT8) {
        uint32_t d0 = (j == 0) ? raw[t].x : raw[t].z;
        uint32_t d1 = (j == 0) ? raw[t].y : raw[t].w;
        h2 q0, q1, q2, q3;
        dq_int8_dword(d0, s2, z2, q0, q1);
        dq_int8_dword(d1, s2, z2, q2, q3);
        b.s01 = q0; b.s23 = q1; b.s45 = q2; b.s67 = q3;
      } else {
        b = __builtin_bit_cast(h8, raw[t]);
      }
      const int koff = t * KSTEP + grp * KPL + 8 * j;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        int m = 16 * mb + nloc;
        h8 a = (h8){0, 0, 0, 0, 0, 0, 0, 0};
        if (m < p.M) a = *(const h8*)(xs + m * XS + koff);
        acc[mb] = mfma16x16x32(a, b, acc[mb]);
      }
    }
  }

  // ---- combine K chunks ----
  // Lane l holds D[m = 16*mb + 4*(l>>4) + r][col = l & 15] of its wave's tile.
  if (p.splits == 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int m = 16 * mb + 4 * grp + r;
        if (m < p.M) tile[m * 64 + col_in_block] = acc[mb][r];
      }
    __syncthreads();
  } else {
    if (row_ok) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int m = 16 * mb + 4 * grp + r;
          if (m < p.M) p.partials[((int64_t)sidx * p.M + m) * p.N + n] = acc[mb][r];
        }
    }
    if (!p.nofence) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
      uint32_t prev = __hip_atomic_fetch_add(p.counters + rb, 1u, __ATOMIC_ACQ_REL,
                                             __HIP_MEMORY_SCOPE_AGENT);
      s_last = (prev == (uint32_t)(p.splits - 1));
    }
    __syncthreads();
    if (!s_last) return;
    if (!p.nofence) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (int idx = tid; idx < p.M * 64; idx += kThreads) {
      int m = idx >> 6, c = idx & 63;
      int nn;
      bool ok;
      if (EPI == EPI_SWIGLU) {
        int j = 32 * rb + (c & 31);
        ok = j < p.F;
        nn = (c >= 32) ? p.F + j : j;
      } else {
        nn = kRowsPerBlock * rb + c;
        ok = nn < p.N;
      }
      float sum = 0.f;
      if (ok) {
        const float* src = p.partials + (int64_t)m * p.N + nn;
        const int64_t stride = (int64_t)p.M * p.N;
        for (int s = 0; s < p.splits; ++s) sum += __builtin_nontemporal_load(src + s * stride);
      }
      tile[idx] = sum;
    }
    if (tid == 0)
      __hip_atomic_store(p.counters + rb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }

  // ---- epilogue ----
  if (EPI == EPI_SWIGLU) {
    for (int idx = tid; idx < p.M * 32; idx += kThreads) {
      int m = idx >> 5, c = idx & 31;
      int j = 32 * rb + c;
      if (j >= p.F) continue;
      float gv = (float)(_Float16)tile[m * 64 + c];
      float uv = (float)(_Float16)tile[m * 64 + 32 + c];
      p.C[(int64_t)m * p.ldc + j] = (_Float16)(silu_f32(gv) * uv);
    }
  } else {
    for (int idx = tid; idx < p.M * 64; idx += kThreads) {
      int m = idx >> 6, c = idx & 63;
      int nn = kRowsPerBlock * rb + c;
      if (nn >= p.N) continue;
      float v = tile[idx];
      if (EPI == EPI_BIAS) v += (float)p.bias[nn];
      p.C[(int64_t)m * p.ldc + nn] = (_Float16)v;
    }
  }
}

template <int FMT, int STEPS, int MB, int EPI>
hipError_t launch_one(const SkinnyKArgs& k, const SkinnyPlan& p, hipStream_t s) {
  hipLaunchKernelGGL((skinny_kernel<FMT, STEPS, MB, EPI>), dim3(p.rblocks, p.splits), dim3(kThreads),
                     p.lds_bytes, s, k);
  return hipGetLastError();
}

template <int FMT, int STEPS, int MB>
hipError_t by_epi(int epi, const SkinnyKArgs& k, const SkinnyPlan& p, hipStream_t s) {
  switch (epi) {
    case EPI_NONE: return launch_one<FMT, STEPS, MB, EPI_NONE>(k, p, s);
    case EPI_BIAS: return launch_one<FMT, STEPS, MB, EPI_BIAS>(k, p, s);
    default: return launch_one<FMT, STEPS, MB, EPI_SWIGLU>(k, p, s);
  }
}

template <int FMT, int STEPS>
hipError_t by_mb(int mb, int epi, const SkinnyKArgs& k, const SkinnyPlan& p, hipStream_t s) {
  switch (mb) {
    case 1: return by_epi<FMT, STEPS, 1>(epi, k, p, s);
    case 2: return by_epi<FMT, STEPS, 2>(epi, k, p, s);
    default: return by_epi<FMT, STEPS, 4>(epi, k, p, s);
  }
}

template <int FMT>
hipError_t by_steps(const SkinnyPlan& p, int epi, const SkinnyKArgs& k, hipStream_t s) {
  switch (p.steps) {
    case 1: return by_mb<FMT, 1>(p.mblocks, epi, k, p, s);
    case 2: return by_mb<FMT, 2>(p.mblocks, epi, k, p, s);
    case 4: return by_mb<FMT, 4>(p.mblocks, epi, k, p, s);
    default: return by_mb<FMT, 8>(p.mblocks, epi, k, p, s);
  }
}

int kpl_of(int fmt) { return fmt == FMT_INT4 ? 32 : (fmt == FMT_INT8 ? 16 : 8); }

}  // namespace

bool skinny_supported(const LinearArgs& a) {
  const int kpl = kpl_of(a.fmt);
  if (a.M < 1 || a.M > 64) return false;
  if (a.K % kpl != 0) return false;                       // whole 16-byte pieces per row
  if (a.fmt != FMT_F16 && (a.g % kpl != 0)) return false;  // one group per piece
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  const int64_t rblocks = (a.epi == EPI_SWIGLU) ? (a.F + 31) / 32 : (a.N + kRowsPerBlock - 1) / kRowsPerBlock;
  if (rblocks * 4 > (int64_t)kWsCounterBytes) return false;  // one counter per row block
  return true;
}

SkinnyPlan skinny_plan(const LinearArgs& a, int num_cus, size_t ws_avail) {
  SkinnyPlan p{};
  const int kstep = 4 * kpl_of(a.fmt);
  p.mblocks = a.M <= 16 ? 1 : (a.M <= 32 ? 2 : 4);
  p.rblocks = (a.epi == EPI_SWIGLU) ? (a.F + 31) / 32 : (a.N + kRowsPerBlock - 1) / kRowsPerBlock;
  // Enough workgroups to give every CU several, using the largest chunk that
  // still does; the activation chunk in LDS stays within 32 KiB.
  const int64_t target = 4LL * num_cus;
  int steps = 8;
  while (steps > 1) {
    int64_t kc = (int64_t)steps * kstep;
    int64_t splits = (a.K + kc - 1) / kc;
    bool lds_ok = (int64_t)a.M * (kc + 8) * 2 <= 32768;
    if (lds_ok && (int64_t)p.rblocks * splits >= target) break;
    steps >>= 1;
  }
  p.steps = steps;
  p.kchunk = steps * kstep;
  p.splits = (a.K + p.kchunk - 1) / p.kchunk;
  p.ws_bytes = p.splits > 1 ? kWsCounterBytes + (size_t)p.splits * a.M * a.N * 4 : 0;
  (void)ws_avail;
  p.lds_bytes = (size_t)a.M * (p.kchunk + 8) * 2 + (size_t)a.M * 64 * 4;
  return p;
}

hipError_t skinny_launch(const LinearArgs& a, const SkinnyPlan& p, void* ws, hipStream_t s) {
  SkinnyKArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.bias = (const _Float16*)a.bias;
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.g = a.g > 0 ? a.g : 1; k.G = a.G; k.F = a.F;
  k.splits = p.splits;
  k.nofence = p.nofence;
  k.gshift = -1;
  for (int b = 0; b < 31; ++b)
    if (k.g == (1 << b)) k.gshift = b;
  if (p.splits > 1) {
    k.counters = (uint32_t*)ws;
    k.partials = (float*)((char*)ws + kWsCounterBytes);
  }
  switch (a.fmt) {
    case FMT_INT4: return by_steps<FMT_INT4>(p, a.epi, k, s);
    case FMT_INT8: return by_steps<FMT_INT8>(p, a.epi, k, s);
    default: return by_steps<FMT_F16>(p, a.epi, k, s);
  }
}

}  // namespace mq
