// Tiled dequant GEMM on v_mfma_f32_32x32x16_f16 (prefill, M >= 17).
//
// Replaces dequant_matmul_int4_fp16 / dequant_matmul_int8_fp16
// (shaders/matmul_dequant_kernel.metal:55-223, :351-479; dispatched at
// src/ops/matmul.mm:1011-1021).  Same contract: C = A . deq(W)^T with fp16
// products accumulated in fp32 and one rounding to fp16 (plus the optional
// bias / SwiGLU epilogue).
//
//  * Workgroup tile BM x 128 (output rows x weight rows) x 64 (K), 4 waves in
//    a 2 x 2 grid; a wave owns (BM/2) x 64 outputs as 32 x 32 MFMA blocks.
//    32x32x16 is used because on gfx950 it runs at about twice the rate of
//    16x16x32 per weight consumed.
//  * Global loads run PF K-tiles ahead of the MFMAs in a register ring (one
//    wave per SIMD leaves room for it): the loads of the activations hit L2,
//    but at roughly a microsecond under load they would otherwise stall every
//    K-tile.  All loads are unconditional buffer loads (out-of-range offsets
//    read zeros), so M / N tails need no branches and the load counter stays
//    exact.
//  * Each K-tile is stored to one of two LDS buffers: activations as they are
//    (int4: re-ordered per 8 to the dequant's operand order), weights
//    dequantized to fp16 with the reference's two roundings.  One barrier per
//    K-tile.
//  * SwiGLU: the 128 weight rows of a tile are 64 gate rows and the matching
//    64 up rows, laid out so that each wave's two 32-column blocks are gate
//    and up of the same 32 outputs: the epilogue has both in one lane.
//  * Workgroups that share a weight tile (same N block, all M blocks) are
//    placed on one XCD, so the tile is fetched into one L2 once.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <type_traits>

#ifndef MQ_GEMM_BK
#define MQ_GEMM_BK 128
#endif

namespace mq {
int g_gemm_pf = 4;
int g_gemm_waves = 8;
int g_gemm_impl = 0;
namespace {

constexpr int BN = 128, BK = MQ_GEMM_BK;
constexpr int LDSW = BK + 8;  // halves per LDS row: conflict-free 16-byte fragment reads

struct GemmKArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros; const _Float16* bias;
  _Float16* C; int64_t ldc;
  int M, N, K, G, F, gshift;
  int nbm, nbn;        // M and N blocks
  int xcd_remap;       // place same-N-block workgroups on one XCD
  uint32_t a_bytes, w_bytes, sz_bytes, z_bytes;
};

__device__ __forceinline__ f16v mfma32(h8 a, h8 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int FMT, int EPI, int BM, int kPF, int NWAVE>
__global__ __launch_bounds__(64 * NWAVE) void gemm_kernel(GemmKArgs p) {
  constexpr int NT = 64 * NWAVE;
  constexpr int WGM = NWAVE / 2;                // waves along M (2 along N, 64 columns each)
  constexpr int WMB = BM / 32 / WGM;            // 32-row blocks per wave
  static_assert(WMB >= 1, "tile too small for the wave count");
  constexpr int APT = BM * BK / 8 / NT;         // 16-byte activation pieces per thread per K-tile
  constexpr int WROW = FMT == FMT_INT4 ? BK / 2 : BK;  // weight bytes per row per K-tile
  constexpr int TPR = NT / BN;                  // threads per weight row
  constexpr int BPT = WROW / TPR;               // weight bytes per thread per K-tile (8, 16 or 32)
  constexpr int KPT = BK / TPR;                 // k per thread per K-tile
  constexpr int WPT = BPT >= 16 ? BPT / 16 : 1; // 16-byte weight loads (or one 8-byte load)
  // one array per buffer: with the buffer index known at compile time the
  // compiler sees that the next tile's stores do not alias this tile's
  // fragment reads and interleaves them with the MFMAs
  __shared__ __align__(16) _Float16 lds_a0[BM * LDSW];
  __shared__ __align__(16) _Float16 lds_a1[BM * LDSW];
  __shared__ __align__(16) _Float16 lds_b0[BN * LDSW];
  __shared__ __align__(16) _Float16 lds_b1[BN * LDSW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  // ---- block coordinates ----
  int id = blockIdx.x;
  if (p.xcd_remap) {  // workgroup i runs on XCD i % 8: give each XCD a contiguous run of ids
    const int per = gridDim.x >> 3;
    id = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  }
  const int nb = id / p.nbm, mb = id - nb * p.nbm;
  const int m0 = mb * BM;

  // ---- loader roles ----
  const rsrc_t ar = make_rsrc(p.A, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  const rsrc_t sr = make_rsrc(p.scales, p.sz_bytes);
  const rsrc_t zr = make_rsrc(p.zeros, p.z_bytes);
  // activations: piece q = tid + NT*e -> row q / PPR, 8-half column q % PPR
  constexpr int PPR = BK / 8;
  uint32_t aoff[APT];
#pragma unroll
  for (int e = 0; e < APT; ++e) {
    const int q = tid + NT * e;
    const int row = m0 + q / PPR;
    aoff[e] = row < p.M ? (uint32_t)((row * p.lda + (q % PPR) * 8) * 2) : kOob;
  }
  // weights: thread = (local row tid / TPR, part tid % TPR of the K-tile)
  const int brow = tid / TPR, bhalf = tid % TPR;
  int grow;
  bool bok;
  if (EPI == EPI_SWIGLU) {
    const int c = nb * 64 + (brow >> 6) * 32 + (brow & 31);  // output column
    bok = c < p.F;
    grow = ((brow >> 5) & 1) ? p.F + c : c;
  } else {
    grow = nb * BN + brow;
    bok = grow < p.N;
  }
  const uint32_t woff = bok ? (uint32_t)(grow * p.ldw) + bhalf * BPT : kOob;
  const uint32_t soff = bok ? (uint32_t)(grow * p.G) * 2 : kOob;

  struct Stage {
    u4 a[APT];
    u4 w[WPT];
    uint16_t s, z;
  };
  const int KT = p.K / BK;
  auto load = [&](int kt, Stage& st) {
    const bool ok = kt < KT;
#pragma unroll
    for (int e = 0; e < APT; ++e) st.a[e] = bload16(ar, ok && aoff[e] != kOob ? aoff[e] + kt * BK * 2 : kOob);
    const uint32_t wo = ok && woff != kOob ? woff + kt * WROW : kOob;
    if (BPT >= 16) {
#pragma unroll
      for (int e = 0; e < WPT; ++e) st.w[e] = bload16_nt(wr, wo == kOob ? kOob : wo + 16 * e);
    } else {
      const uint64_t v = bload8_nt(wr, wo);
      st.w[0] = (u4){(uint32_t)v, (uint32_t)(v >> 32), 0u, 0u};
    }
    const int g = ((kt * BK + bhalf * KPT) >> p.gshift);
    const uint32_t so = ok && soff != kOob ? soff + (uint32_t)g * 2 : kOob;
    st.s = bload2h(sr, so);
    st.z = bload2h(zr, so);
  };
  auto store = [&](auto bufc, const Stage& st) {
    constexpr int buf = decltype(bufc)::value;
    _Float16* as = buf ? lds_a1 : lds_a0;
#pragma unroll
    for (int e = 0; e < APT; ++e) {
      const int q = tid + NT * e;
      u4 v = st.a[e];
      if (FMT == FMT_INT4) v = perm8_int4(v);
      *(u4*)(as + (q / PPR) * LDSW + (q % PPR) * 8) = v;
    }
    _Float16* bs = (buf ? lds_b1 : lds_b0) + brow * LDSW + bhalf * KPT;
    const h2 s2 = as_h2((uint32_t)st.s * 0x10001u);
    const h2 z2 = as_h2((uint32_t)st.z * 0x10001u);
    if (FMT == FMT_INT4) {
#pragma unroll
      for (int e = 0; e < WPT; ++e) {
        const u4 v = st.w[e];
        *(h8*)(bs + 32 * e + 0) = dq_int4_dword_perm(v.x, s2, z2);
        *(h8*)(bs + 32 * e + 8) = dq_int4_dword_perm(v.y, s2, z2);
        if (BPT >= 16) {
          *(h8*)(bs + 32 * e + 16) = dq_int4_dword_perm(v.z, s2, z2);
          *(h8*)(bs + 32 * e + 24) = dq_int4_dword_perm(v.w, s2, z2);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < WPT; ++e) {
        const u4 v = st.w[e];
        h2 q[8];
        dq_int8_dword(v.x, s2, z2, q[0], q[1]);
        dq_int8_dword(v.y, s2, z2, q[2], q[3]);
        dq_int8_dword(v.z, s2, z2, q[4], q[5]);
        dq_int8_dword(v.w, s2, z2, q[6], q[7]);
        h8 b0, b1;
        b0.s01 = q[0]; b0.s23 = q[1]; b0.s45 = q[2]; b0.s67 = q[3];
        b1.s01 = q[4]; b1.s23 = q[5]; b1.s45 = q[6]; b1.s67 = q[7];
        *(h8*)(bs + 16 * e) = b0;
        *(h8*)(bs + 16 * e + 8) = b1;
      }
    }
  };

  f16v acc[WMB][2];
#pragma unroll
  for (int i = 0; i < WMB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f16v){};

  const int fr = lane & 31, fk = 8 * (lane >> 5);  // fragment row/col and k offset
  auto compute = [&](auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const _Float16* as = (buf ? lds_a1 : lds_a0) + (wm * 32 * WMB + fr) * LDSW + fk;
    const _Float16* bs = (buf ? lds_b1 : lds_b0) + (wn * 64 + fr) * LDSW + fk;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      h8 a[WMB], b[2];
#pragma unroll
      for (int i = 0; i < WMB; ++i) a[i] = *(const h8*)(as + i * 32 * LDSW + kk * 16);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *(const h8*)(bs + j * 32 * LDSW + kk * 16);
#pragma unroll
      for (int i = 0; i < WMB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    }
  };

  // ---- pipeline: loads kPF K-tiles ahead, LDS double buffer ----
  // The loop is unrolled by kPF (even) so that ring slot and LDS buffer are
  // compile-time constants in every step.
  static_assert(kPF % 2 == 0, "ring depth must be even (LDS buffer parity)");
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  Stage st[kPF];
#pragma unroll
  for (int s = 0; s < kPF; ++s) load(s, st[s]);
  store(I0{}, st[0]);
  __syncthreads();
  // One K-tile per step, branch-free so that the MFMAs of this tile, the
  // dequant and LDS stores of the next and the loads kPF tiles ahead form one
  // scheduling region; the group barriers below interleave them (the MFMA
  // pipe then runs while the VALU dequantizes).  The last step stores a tile
  // of zeros (loads past K read zeros) into the idle buffer: harmless.
  auto kstep = [&](auto sc, int kt) {
    constexpr int s = decltype(sc)::value;
    using B = std::integral_constant<int, s & 1>;
    using NB = std::integral_constant<int, (s & 1) ^ 1>;
    load(kt + kPF, st[s]);  // slot s held tile kt, already in LDS
    compute(B{});
    store(NB{}, st[(s + 1) % kPF]);
#pragma unroll
    for (int i = 0; i < 4 * WMB * 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
    }
    __syncthreads();
  };
  for (int kt0 = 0; kt0 < KT; kt0 += kPF) {  // KT is a multiple of kPF
    kstep(std::integral_constant<int, 0>{}, kt0 + 0);
    kstep(std::integral_constant<int, 1>{}, kt0 + 1);
    if constexpr (kPF > 2) {
      kstep(std::integral_constant<int, 2 % kPF>{}, kt0 + 2);
      kstep(std::integral_constant<int, 3 % kPF>{}, kt0 + 3);
    }
    if constexpr (kPF > 4) {
      kstep(std::integral_constant<int, 4 % kPF>{}, kt0 + 4);
      kstep(std::integral_constant<int, 5 % kPF>{}, kt0 + 5);
    }
    if constexpr (kPF > 6) {
      kstep(std::integral_constant<int, 6 % kPF>{}, kt0 + 6);
      kstep(std::integral_constant<int, 7 % kPF>{}, kt0 + 7);
    }
  }
  (void)I1{};

  // ---- epilogue ----
#pragma unroll
  for (int i = 0; i < WMB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) mfma_result_fence16(acc[i][j]);
  // lane holds D[row = 8*(v/4) + 4*(lane/32) + v%4][col = lane%32] of each block
  const int rbase = m0 + wm * 32 * WMB + 4 * (lane >> 5);  // wave rows wm*32*WMB .. +32*WMB
  if (EPI == EPI_SWIGLU) {
    const int col = nb * 64 + wn * 32 + fr;
    if (col < p.F) {
#pragma unroll
      for (int i = 0; i < WMB; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = rbase + 32 * i + 8 * (v >> 2) + (v & 3);
          if (row < p.M) {
            const float gv = (float)(_Float16)acc[i][0][v];
            const float uv = (float)(_Float16)acc[i][1][v];
            p.C[(int64_t)row * p.ldc + col] = (_Float16)(silu_f32(gv) * uv);
          }
        }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = nb * BN + wn * 64 + 32 * j + fr;
      if (col >= p.N) continue;
      const float bv = (EPI == EPI_BIAS) ? (float)p.bias[col] : 0.f;
#pragma unroll
      for (int i = 0; i < WMB; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = rbase + 32 * i + 8 * (v >> 2) + (v & 3);
          if (row < p.M) p.C[(int64_t)row * p.ldc + col] = (_Float16)(acc[i][j][v] + bv);
        }
    }
  }
}

template <int FMT, int EPI, int BM, int NWAVE>
hipError_t launch4(const GemmKArgs& k, int pf, int nwg, hipStream_t s) {
  switch (pf) {
    case 8: hipLaunchKernelGGL((gemm_kernel<FMT, EPI, BM, 8, NWAVE>), dim3(nwg), dim3(64 * NWAVE), 0, s, k); break;
    case 4: hipLaunchKernelGGL((gemm_kernel<FMT, EPI, BM, 4, NWAVE>), dim3(nwg), dim3(64 * NWAVE), 0, s, k); break;
    default: hipLaunchKernelGGL((gemm_kernel<FMT, EPI, BM, 2, NWAVE>), dim3(nwg), dim3(64 * NWAVE), 0, s, k); break;
  }
  return hipGetLastError();
}

template <int FMT, int EPI, int BM>
hipError_t launch3(const GemmKArgs& k, int pf, int nwg, hipStream_t s) {
  if constexpr (BM == 128) {
    if (g_gemm_waves == 8) return launch4<FMT, EPI, BM, 8>(k, pf, nwg, s);
  }
  return launch4<FMT, EPI, BM, 4>(k, pf, nwg, s);
}

template <int FMT, int EPI>
hipError_t launch2(const GemmKArgs& k, int bm, int pf, int nwg, hipStream_t s) {
  return bm == 128 ? launch3<FMT, EPI, 128>(k, pf, nwg, s) : launch3<FMT, EPI, 64>(k, pf, nwg, s);
}

template <int FMT>
hipError_t launch1(const GemmKArgs& k, int epi, int bm, int pf, int nwg, hipStream_t s) {
  if (epi == EPI_NONE) return launch2<FMT, EPI_NONE>(k, bm, pf, nwg, s);
  if (epi == EPI_BIAS) return launch2<FMT, EPI_BIAS>(k, bm, pf, nwg, s);
  return launch2<FMT, EPI_SWIGLU>(k, bm, pf, nwg, s);
}

// ring depth: the preferred one if it divides the K-tile count, else the
// largest even one that does (K is a multiple of 2 K-tiles)
int pf_for(int kt) {
  if (kt % g_gemm_pf == 0) return g_gemm_pf;
  for (int pf : {8, 4, 2})
    if (kt % pf == 0) return pf;
  return 0;
}

int gshift_of(const LinearArgs& a) {
  if (a.G == 1) return 31;
  for (int b = 0; b < 31; ++b)
    if (a.g == (1 << b)) return b;
  return -1;
}

}  // namespace

bool gemm_supported(const LinearArgs& a) {
  if (a.fmt != FMT_INT4 && a.fmt != FMT_INT8) return false;
  if (a.K % (2 * BK) != 0) return false;  // an even number of K-tiles
  if (a.G != 1 && (gshift_of(a) < 0 || a.g < BK / 2)) return false;  // a thread's 32 k lie in one group
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  const int64_t lim = (int64_t)1 << 31;
  if (((int64_t)(a.M - 1) * a.lda + a.K) * 2 >= lim) return false;
  if ((int64_t)a.N * a.ldw >= lim || (int64_t)a.N * a.G * 2 >= lim) return false;
  return true;
}

hipError_t gemm_launch(const LinearArgs& a, hipStream_t s) {
  GemmKArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.bias = (const _Float16*)a.bias;
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.G = a.G; k.F = a.F;
  k.gshift = gshift_of(a);
  const int bm = a.M <= 64 ? 64 : 128;
  k.nbm = (a.M + bm - 1) / bm;
  k.nbn = a.epi == EPI_SWIGLU ? (a.F + 63) / 64 : (a.N + BN - 1) / BN;
  const int nwg = k.nbm * k.nbn;
  k.xcd_remap = (nwg % 8 == 0) ? 1 : 0;
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  k.w_bytes = (uint32_t)((int64_t)a.N * a.ldw);
  k.sz_bytes = (uint32_t)(((int64_t)a.N * a.G * 2 + 3) & ~(int64_t)3);
  k.z_bytes = a.zeros ? k.sz_bytes : 0u;
  const int pf = pf_for(a.K / BK);
  if (a.fmt == FMT_INT4) return launch1<FMT_INT4>(k, a.epi, bm, pf, nwg, s);
  return launch1<FMT_INT8>(k, a.epi, bm, pf, nwg, s);
}

}  // namespace mq
