// Prefill dequant GEMM with weights dequantized straight into MFMA operand
// registers (v_mfma_f32_32x32x16_f16, M >= 17).
//
// Replaces dequant_matmul_int4_fp16 / dequant_matmul_int8_fp16
// (shaders/matmul_dequant_kernel.metal:55-223, :351-479; dispatched at
// src/ops/matmul.mm:1011-1021).  Same contract as the LDS-staged kernel in
// mq_gemm.hip: C = A . deq(W)^T, fp16 products accumulated in fp32, one
// rounding to fp16, optional bias or SwiGLU epilogue.
//
//  * A wave owns 32 weight rows (SwiGLU: half the waves own gate rows, the
//    other half the matching up rows; the epilogue pairs them through LDS)
//    across all BM output rows of the workgroup, so every weight is
//    loaded and dequantized exactly once per workgroup, by the lane that feeds
//    it to the MFMA: weights never pass through LDS.
//  * Only the activation tile (BM x 128 k) is shared through LDS, double
//    buffered, one barrier per K-tile.  Per MFMA a wave reads one 1 KiB A
//    fragment from LDS for BM/32 = 4 MFMAs per B fragment, half the LDS reads
//    per MFMA of a 2 x 4 wave grid that also reads B from LDS.
//  * K order inside a K-tile is permuted (the sum does not care): lane half h
//    at k-step kk takes the 8 k starting at byte (kk/4)*32 + h*16 + (kk%4)*4
//    of the int4 row (int8: (kk/2)*32 + h*16 + (kk%2)*8), so one 16-byte load
//    of the two halves covers 32 contiguous bytes of each weight row.  The A
//    fragment is read from the same k.
//  * Two waves share each weight slice, one per half of a K-tile's eight
//    k-steps (KS = 2): every SIMD holds two waves, so one wave's LDS and load
//    waits overlap the other's MFMAs, and no weight is dequantized twice.  The
//    two partial sums are added once, through LDS, after the K loop.  With one
//    wave per slice (and one wave per SIMD) the same kernel took 47 us at the
//    Llama-3.2-3B QKV shape (M = 512) against 35 us with two; a four-way
//    split (four waves per SIMD, 8-byte int4 loads) took 44 us and was
//    removed.
//  * Global loads run PF K-tiles ahead in a register ring; the next tile's
//    weights are dequantized while this tile's MFMAs run.
//  * Workgroups sharing a weight slice (same N block, all M blocks) are placed
//    on one XCD.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <type_traits>


namespace mq {
namespace {

constexpr int BK = 128;
constexpr int LDSW = BK + 8;  // halves per LDS row: conflict-free 16-byte fragment reads

struct GemmRArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros; const _Float16* bias;
  _Float16* C; int64_t ldc;
  int M, N, K, G, F, gshift;
  int nbm, nbn;
  int xcd_remap;
  uint32_t a_bytes, w_bytes, sz_bytes, z_bytes;
};

__device__ __forceinline__ f16v mfma32(h8 a, h8 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// k offset (halves) inside the K-tile of lane half h at k-step kk
template <int FMT>
__device__ __forceinline__ constexpr int kcol(int h, int kk) {
  return FMT == FMT_INT4 ? (kk >> 2) * 64 + h * 32 + (kk & 3) * 8 : (kk >> 1) * 32 + h * 16 + (kk & 1) * 8;
}

template <int FMT, int EPI, int BM, int NW, int PF, int KS>
__global__ __launch_bounds__(64 * NW * KS) void gemmr_kernel(GemmRArgs p) {
  constexpr int NT = 64 * NW * KS;
  constexpr int MB = BM / 32;                          // A blocks per wave
  constexpr int NBB = 1;                               // B blocks (32 weight rows) per wave
  constexpr int APT = BM * BK / 8 / NT;                // 16-byte activation pieces per thread per K-tile
  constexpr int KKW = 8 / KS;                          // k-steps per wave per K-tile
  constexpr int NDW = FMT == FMT_INT4 ? KKW : 2 * KKW; // weight dwords per lane per B block per K-tile
  constexpr int WL = NDW / 4;                          // 16-byte weight loads per lane
  static_assert(KS == 2 && WL >= 1, "two k-halves, whole 16-byte weight loads");
  constexpr int WROW = FMT == FMT_INT4 ? BK / 2 : BK;  // weight bytes per row per K-tile
  static_assert(APT >= 1, "tile too small");
  __shared__ __align__(16) _Float16 lds_a0[BM * LDSW];
  __shared__ __align__(16) _Float16 lds_a1[BM * LDSW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, h = lane >> 5;
  const int wc = w % NW, ks = w / NW;  // column slice and k-half of this wave

  int id = blockIdx.x;
  if (p.xcd_remap) {  // workgroup i runs on XCD i % 8: give each XCD a contiguous run of ids
    const int per = gridDim.x >> 3;
    id = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  }
  const int nb = id / p.nbm, mb = id - nb * p.nbm;
  const int m0 = mb * BM;

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
  // weights: B block j of this wave, column fr
  // output column; SwiGLU: waves wc < NW/2 own gate rows, wave wc + NW/2 the
  // matching up rows, and the workgroup covers 16*NW outputs
  constexpr int NH = NW / 2;
  const int col = EPI == EPI_SWIGLU ? nb * 32 * NH + (wc % NH) * 32 + fr : nb * 32 * NW + wc * 32 + fr;
  const bool is_up = EPI == EPI_SWIGLU && wc >= NH;
  uint32_t woff[NBB], soff[NBB];
#pragma unroll
  for (int j = 0; j < NBB; ++j) {
    const bool ok = col < (EPI == EPI_SWIGLU ? p.F : p.N);
    const int grow = (is_up ? p.F + col : col) + j * 32;
    // first byte of this lane's k-steps ks*KKW .. : int4 k-step kk sits at
    // (kk/4)*32 + h*16 + (kk%4)*4, int8 at (kk/2)*32 + h*16 + (kk%2)*8
    const int kk0 = ks * KKW;
    const int b0 = FMT == FMT_INT4 ? (kk0 >> 2) * 32 + (kk0 & 3) * 4 : (kk0 >> 1) * 32;
    woff[j] = ok ? (uint32_t)(grow * p.ldw) + b0 + h * 16 : kOob;
    soff[j] = ok ? (uint32_t)(grow * p.G) * 2 : kOob;
  }

  struct Stage {
    u4 a[APT];
    uint32_t w[NBB][NDW];
    uint16_t s[NBB], z[NBB];
  };
  const int KT = p.K / BK;
  // The K-tile offset is uniform: it goes in the loads' scalar offset, so a
  // load costs no per-lane VALU.  Per-lane offsets are kOob for rows past M or
  // N (those loads read zeros whatever the scalar offset); tiles past K (the
  // ring's last PF loads, never used) re-read the last tile.
  // Weight loads are cached normally, not streamed: the workgroups of the
  // other M blocks read the same slice at about the same time on the same XCD
  // (33.9 -> 31.8 us at the Llama-3.2-3B QKV shape).
  auto load = [&](int kt, Stage& st) {
    const int kc = kt < KT ? kt : KT - 1;
    const uint32_t sa = (uint32_t)(kc * BK * 2);
#pragma unroll
    for (int e = 0; e < APT; ++e)
      st.a[e] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(ar, aoff[e], sa, 0));
    const uint32_t sw = (uint32_t)(kc * WROW);
    const uint32_t g2 = (uint32_t)((kc * BK) >> p.gshift) * 2;
#pragma unroll
    for (int j = 0; j < NBB; ++j) {
#pragma unroll
      for (int e = 0; e < WL; ++e) {
        const u4 v = __builtin_bit_cast(
            u4, __builtin_amdgcn_raw_buffer_load_b128(wr, woff[j] == kOob ? kOob : woff[j] + 32 * e, sw, 0));
        st.w[j][4 * e] = v.x; st.w[j][4 * e + 1] = v.y; st.w[j][4 * e + 2] = v.z; st.w[j][4 * e + 3] = v.w;
      }
      st.s[j] = __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(sr, soff[j], g2, 0));
      st.z[j] = __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(zr, soff[j], g2, 0));
    }
  };
  auto store_a = [&](auto bufc, const Stage& st) {
    constexpr int buf = decltype(bufc)::value;
    _Float16* as = buf ? lds_a1 : lds_a0;
#pragma unroll
    for (int e = 0; e < APT; ++e) {
      const int q = tid + NT * e;
      u4 v = st.a[e];
      if (FMT == FMT_INT4) v = perm8_int4(v);
      *(u4*)(as + (q / PPR) * LDSW + (q % PPR) * 8) = v;
    }
  };
  // dequantized B fragments of one K-tile: [k-step][block]
  h8 bq0[KKW][NBB], bq1[KKW][NBB];
  // nibble masks in VGPRs and the fp16 1024 pair in an SGPR: one v_and_or_b32
  // per nibble pair instead of an AND and an OR with literal operands
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u;
  asm volatile("" : "+v"(mlo), "+v"(mhi));
  const uint32_t magic = 0x64006400u;
  auto dequant = [&](auto bufc, const Stage& st) {
    constexpr int buf = decltype(bufc)::value;
    auto& bq = buf ? bq1 : bq0;
#pragma unroll
    for (int j = 0; j < NBB; ++j) {
      const h2 s2 = as_h2((uint32_t)st.s[j] * 0x10001u);
      const h2 z2 = as_h2((uint32_t)st.z[j] * 0x10001u);
#pragma unroll
      for (int t = 0; t < KKW; ++t) {
        if (FMT == FMT_INT4) {
          bq[t][j] = dq_int4_dword_perm_r(st.w[j][t], s2, z2, mlo, mhi, magic);
        } else {
          h2 q[4];
          dq_int8_dword(st.w[j][2 * t], s2, z2, q[0], q[1]);
          dq_int8_dword(st.w[j][2 * t + 1], s2, z2, q[2], q[3]);
          h8 b;
          b.s01 = q[0]; b.s23 = q[1]; b.s45 = q[2]; b.s67 = q[3];
          bq[t][j] = b;
        }
      }
    }
  };

  f16v acc[MB][NBB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NBB; ++j) acc[i][j] = (f16v){};

  auto compute = [&](auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const _Float16* as = (buf ? lds_a1 : lds_a0) + fr * LDSW;
    auto& bq = buf ? bq1 : bq0;
#pragma unroll
    for (int t = 0; t < KKW; ++t) {
      const int kk = ks * KKW + t;
      const int kc = kcol<FMT>(h, kk);
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const h8 a = *(const h8*)(as + i * 32 * LDSW + kc);
#pragma unroll
        for (int j = 0; j < NBB; ++j) acc[i][j] = mfma32(a, bq[t][j], acc[i][j]);
      }
    }
  };

  // ---- pipeline ----
  // Tile t sits in ring slot t % PF.  Step kt: MFMAs of tile kt (LDS buffer
  // kt & 1, B fragments bq[kt & 1]); tile kt+1's activations go to the other
  // LDS buffer and its weights are dequantized into the other bq; its slot is
  // then free and takes tile kt+1+PF.  The loop is unrolled by lcm(2, PF) so
  // that slots and buffers are compile-time constants.
  constexpr int U = PF % 2 == 0 ? PF : 2 * PF;
  using I0 = std::integral_constant<int, 0>;
  Stage st[PF];
#pragma unroll
  for (int s = 0; s < PF; ++s) load(s, st[s]);
  store_a(I0{}, st[0]);
  dequant(I0{}, st[0]);
  load(PF, st[0]);
  __syncthreads();
  auto kstep = [&](auto sc, int kt) {
    constexpr int s = decltype(sc)::value;  // kt % U
    using B = std::integral_constant<int, s & 1>;
    using NB = std::integral_constant<int, (s & 1) ^ 1>;
    constexpr int ns = (s + 1) % PF;
    compute(B{});
    store_a(NB{}, st[ns]);
    dequant(NB{}, st[ns]);
    load(kt + 1 + PF, st[ns]);
    __syncthreads();
  };
  for (int kt0 = 0; kt0 < KT; kt0 += U) {  // KT is a multiple of U
    kstep(std::integral_constant<int, 0>{}, kt0 + 0);
    kstep(std::integral_constant<int, 1>{}, kt0 + 1);
    if constexpr (U > 2) {
      kstep(std::integral_constant<int, 2>{}, kt0 + 2);
      kstep(std::integral_constant<int, 3>{}, kt0 + 3);
    }
    if constexpr (U > 4) {
      kstep(std::integral_constant<int, 4>{}, kt0 + 4);
      kstep(std::integral_constant<int, 5>{}, kt0 + 5);
    }
  }

  // ---- epilogue ----
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NBB; ++j) mfma_result_fence16(acc[i][j]);
  // The two k-halves' partial sums meet through LDS (the activation buffers
  // are free now).  Wave ks finishes blocks i with i / (MB/2) == ks: it
  // receives the other wave's partials of those blocks and hands over its own
  // of the rest, so both waves share the reduction and the stores.  Block i
  // of column slice wc sits in buffer i & 1 at 16 KiB * (i >> 1).
  static_assert(KS == 2 && NBB == 1 && MB % 2 == 0, "the epilogue pairs two k-halves");
  static_assert(BM * LDSW * 2 >= (MB / 2) * NW * 16 * 64 * 4, "reduction does not fit");
  auto mine = [&](int i) { return i / (MB / 2) == ks; };
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MB; ++i)
    if (!mine(i)) {
      float* r = (float*)(i & 1 ? lds_a1 : lds_a0) + ((i >> 1) * NW + wc) * 16 * 64 + lane;
#pragma unroll
      for (int v = 0; v < 16; ++v) r[v * 64] = acc[i][0][v];
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MB; ++i)
    if (mine(i)) {
      const float* r = (const float*)(i & 1 ? lds_a1 : lds_a0) + ((i >> 1) * NW + wc) * 16 * 64 + lane;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][0][v] += r[v * 64];
    }
  // lane holds D[row = 8*(v/4) + 4*(lane/32) + v%4][col = lane%32] of each block
  const int rbase = m0 + 4 * h;
  if constexpr (EPI == EPI_SWIGLU) {
    // up waves hand their finished blocks to the matching gate waves (same
    // LDS slots as the k-half exchange, which every wave has read by now)
    __syncthreads();
    if (is_up) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
        if (mine(i)) {
          float* r = (float*)(i & 1 ? lds_a1 : lds_a0) + ((i >> 1) * NW + wc - NH) * 16 * 64 + lane;
#pragma unroll
          for (int v = 0; v < 16; ++v) r[v * 64] = acc[i][0][v];
        }
    }
    __syncthreads();
    if (!is_up && col < p.F) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
        if (mine(i)) {
          const float* r = (const float*)(i & 1 ? lds_a1 : lds_a0) + ((i >> 1) * NW + wc) * 16 * 64 + lane;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int row = rbase + 32 * i + 8 * (v >> 2) + (v & 3);
            if (row < p.M) {
              const float gv = (float)(_Float16)acc[i][0][v];
              const float uv = (float)(_Float16)r[v * 64];
              p.C[(int64_t)row * p.ldc + col] = (_Float16)(silu_f32(gv) * uv);
            }
          }
        }
    }
  } else if (col < p.N) {
    const float bv = (EPI == EPI_BIAS) ? (float)p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < MB; ++i)
      if (mine(i)) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = rbase + 32 * i + 8 * (v >> 2) + (v & 3);
          if (row < p.M) p.C[(int64_t)row * p.ldc + col] = (_Float16)(acc[i][0][v] + bv);
        }
      }
  }
}

template <int FMT, int EPI>
hipError_t launch2(const GemmRArgs& k, int bm, int nwg, hipStream_t s) {
  // SwiGLU: two column waves (one gate, one up) per k-half, 32 outputs per
  // workgroup: 592 workgroups at the Qwen2.5-7B gate+up shape balance better
  // over 256 CUs than 296 of 64 outputs (59.6 against 64.2 us at M = 64)
  constexpr int NW = EPI == EPI_SWIGLU ? 2 : 4, KS = 2;
  if (bm == 128)
    hipLaunchKernelGGL((gemmr_kernel<FMT, EPI, 128, NW, 2, KS>), dim3(nwg), dim3(64 * KS * NW), 0, s, k);
  else
    hipLaunchKernelGGL((gemmr_kernel<FMT, EPI, 64, NW, 2, KS>), dim3(nwg), dim3(64 * KS * NW), 0, s, k);
  return hipGetLastError();
}

template <int FMT>
hipError_t launch1(const GemmRArgs& k, int epi, int bm, int nwg, hipStream_t s) {
  if (epi == EPI_NONE) return launch2<FMT, EPI_NONE>(k, bm, nwg, s);
  if (epi == EPI_BIAS) return launch2<FMT, EPI_BIAS>(k, bm, nwg, s);
  return launch2<FMT, EPI_SWIGLU>(k, bm, nwg, s);
}

int gshift_of(const LinearArgs& a) {
  if (a.G == 1) return 31;
  for (int b = 0; b < 31; ++b)
    if (a.g == (1 << b)) return b;
  return -1;
}

}  // namespace

bool gemmr_supported(const LinearArgs& a) {
  if (a.fmt != FMT_INT4 && a.fmt != FMT_INT8) return false;
  if (a.K % BK != 0 || (a.K / BK) % 2 != 0) return false;
  // a lane's k within a K-tile span the whole tile: one group per K-tile
  if (a.G != 1 && (gshift_of(a) < 0 || a.g < BK)) return false;
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  const int64_t lim = (int64_t)1 << 31;
  if (((int64_t)(a.M - 1) * a.lda + a.K) * 2 >= lim) return false;
  if ((int64_t)a.N * a.ldw >= lim || (int64_t)a.N * a.G * 2 >= lim) return false;
  return true;
}

hipError_t gemmr_launch(const LinearArgs& a, hipStream_t s) {
  GemmRArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.bias = (const _Float16*)a.bias;
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.G = a.G; k.F = a.F;
  k.gshift = gshift_of(a);
  const int bm = a.M <= 64 ? 64 : 128;
  const int nw = a.epi == EPI_SWIGLU ? 2 : 4;
  k.nbm = (a.M + bm - 1) / bm;
  k.nbn = a.epi == EPI_SWIGLU ? (a.F + 16 * nw - 1) / (16 * nw) : (a.N + 32 * nw - 1) / (32 * nw);
  const int nwg = k.nbm * k.nbn;
  k.xcd_remap = (nwg % 8 == 0) ? 1 : 0;
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  k.w_bytes = (uint32_t)((int64_t)a.N * a.ldw);
  k.sz_bytes = (uint32_t)(((int64_t)a.N * a.G * 2 + 3) & ~(int64_t)3);
  k.z_bytes = a.zeros ? k.sz_bytes : 0u;
  if (a.fmt == FMT_INT4) return launch1<FMT_INT4>(k, a.epi, bm, nwg, s);
  return launch1<FMT_INT8>(k, a.epi, bm, nwg, s);
}

}  // namespace mq
