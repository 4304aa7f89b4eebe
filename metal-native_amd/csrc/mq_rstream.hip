// Register-streamed row-block decode GEMV for skinny activations whose
// activation rows do not fit in LDS whole (int4 weights, 3 <= M <= 16, long
// K; the Qwen2.5-7B down-proj at M = 5..16 is its main case).
//
// Replaces, like mq_rows.hip and mq_gemv.hip, the reference's M<=8 routes
// (shaders/matmul_dequant_kernel.metal:229-345 and :485-576, dispatched at
// src/ops/matmul.mm:946-1009), computing every row of A.
//
// Structure (one launch, no workspace, no barrier before the stream):
//  * One workgroup of 12 wavefronts per CU owns R consecutive output rows
//    (SwiGLU: R output columns = R gate + R up weight rows) over the whole of
//    K: TW <= 4 row tiles of RPW >= 4 weight rows (the last one may be partly
//    empty).  A tile's RPW rows x S = 16/RPW K shifts are the 16 columns of
//    the B operand of v_mfma_f32_16x16x32_f16; the A operand holds activation
//    row i % RPW at K shift i / RPW (M <= RPW), and the result for
//    (activation i, weight row r) is sum_s D[s*RPW + i][s*RPW + r].
//  * The workgroup's TW x KS units (tile, K step) are numbered step-major and
//    wave w takes the contiguous range [w*U/NW, (w+1)*U/NW): the waves split
//    K, each touching every tile, and keep one accumulator per tile.
//  * Per K step a wave brings the step's activation pieces into a ring of 3
//    LDS slots of its own (4 KiB each) by coalesced direct-to-LDS loads and
//    reads its MFMA fragments from there (permuted to the weights' unpack
//    order in registers); per unit each lane loads its 16 weight bytes into
//    a register ring of the same 3 steps.  The scales and zeros of the
//    wave's groups (its tile rows x the groups of its K range) are staged in
//    a per-wave LDS table at the start.  All loads are unconditional
//    (outside the wave's range they use out-of-range offsets), so the load
//    counter is exact, and no barrier precedes the stream.
//  * At the end each wave folds the K shifts of its accumulators through a
//    scratch in its own first activation slot into per-tile partials; after
//    one barrier every output sums the waves' partials in wave order
//    (deterministic; a wave that did not touch a tile contributes +0),
//    applies the epilogue and stores fp16.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <algorithm>

namespace mq {
namespace {

constexpr int kRsNW = 12;       // wavefronts per workgroup (3 per SIMD)
constexpr int kRsSteps = 3;     // K steps in flight per wave (activation ring: 12 KiB of LDS per wave)
constexpr int kRsSzEnt = 256;   // scale-table entries per wave (tile rows x groups of its K range)

struct RsArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros;
  EpiArgs ep;     // element-wise epilogue (kernels without SwiGLU)
  _Float16* C; int64_t ldc;
  int M, K, N, F, G, gshift;
  int R;          // output rows (SwiGLU: output columns) per workgroup
  int TW;         // row tiles per workgroup
  int KS;         // K steps per row
  uint32_t a_bytes, s_bytes, z_bytes;
};

template <int I, int NW, int NJ>
__device__ __forceinline__ u4 (&rs_aslot())[NW][NJ * 64] {
  __shared__ u4 a[NW][NJ * 64];
  return a;
}

template <int FMT, int EPI, int RPW, int TWM, int NW>
__global__ __launch_bounds__(64 * NW) void rstream_kernel(RsArgs p) {
  constexpr int S = 16 / RPW;
  constexpr int KPL = FmtTraits<FMT>::KPL;       // k per 16-byte weight piece
  constexpr int KSTEP = 4 * KPL * S;             // k per row per unit
  constexpr int NJ = KPL / 8;                    // MFMAs per unit
  constexpr int HALF = RPW / 2;
  constexpr int BPK2 = FMT == FMT_INT4 ? 1 : 2;  // 2 x bytes per k
  constexpr int L = kRsSteps;                    // K steps in flight
  constexpr int NT = 64 * NW;
  constexpr int SZE = kRsSzEnt / 64;             // scale-table entries staged per lane
  static_assert(FMT == FMT_INT4, "int4 weights (the activation swizzle assumes 16 pieces per K shift)");
  static_assert(EPI != EPI_SWIGLU || RPW >= 2, "a SwiGLU tile pairs gate and up rows");
  static_assert(L == 3, "the ring is unrolled by 3");
  static_assert(256 + TWM * RPW * RPW <= NJ * 64 * 4, "fold scratch and partials fit in a wave's first slot");
  __shared__ uint32_t szt[NW][kRsSzEnt];          // per wave: s | z << 16, [table row][group - g0]

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x;
  const int M = p.M, TW = p.TW, KS = p.KS;
  const int nl = lane & 15, gi = lane >> 4;
  const int r = nl % RPW, sh = nl / RPW;          // weight row in tile, K shift
  const int klane = sh * 4 * KPL + gi * KPL;      // this lane's k within a unit

  // ---- this workgroup's rows (as mq_rows.hip): plain lr = t*RPW + r; SwiGLU
  // gate column c = t*HALF + r % HALF, weight rows c and F + c ----
  const int row0 = b * p.R;
  int valid;
  uint32_t span;
  if (EPI == EPI_SWIGLU) {
    valid = max(0, min(p.R, p.F - row0));
    span = (uint32_t)((p.F + valid) * p.ldw);
  } else {
    valid = max(0, min(p.R, p.N - row0));
    span = (uint32_t)(valid * p.ldw);
  }
  // weight row (relative to row0) of table row tr = t*RPW + rr, or -1
  auto lrow_of = [&](int t, int rr) -> int {
    if (t >= TW) return -1;
    if (EPI == EPI_SWIGLU) {
      const int c = t * HALF + (rr % HALF);
      return c < valid ? (rr < HALF ? c : p.F + c) : -1;
    }
    const int lr = t * RPW + rr;
    return lr < valid ? lr : -1;
  };
  const rsrc_t wr = make_rsrc(p.W + (int64_t)row0 * p.ldw, span);
  const rsrc_t ar = make_rsrc(p.A, p.a_bytes);
  const rsrc_t sr = make_rsrc(p.scales, p.s_bytes);
  const rsrc_t zr = make_rsrc(p.zeros, p.z_bytes);
  constexpr uint32_t kOobPart = 0x40000000u;   // a sum of two parts still fails the range check
  uint32_t lvo[TWM];                           // per tile: the lane's weight offset (lane part)
#pragma unroll
  for (int t = 0; t < TWM; ++t) {
    const int lr = lrow_of(t, r);
    lvo[t] = lr < 0 ? kOobPart : (uint32_t)(lr * p.ldw) + (uint32_t)(klane * BPK2 / 2);
  }
  const int gsh = p.gshift;

  // ---- unit range ----
  const int U = TW * KS;
  const int u0 = (w * U) / NW, u1 = ((w + 1) * U) / NW;
  const int js = u0 / TW, je = u1 > u0 ? (u1 - 1) / TW : js - 1;   // steps touched: [js, je]

  // ---- scale table of the wave's groups (loads first: the load counter
  // completes in order) ----
  const int g0 = gsh >= 31 ? 0 : (js * KSTEP) >> gsh;
  const int g1 = je < js ? g0 : (gsh >= 31 ? 0 : min(((je + 1) * KSTEP - 1) >> gsh, p.G - 1));
  const int ngw = g1 - g0 + 1;                  // groups per table row
  const int nent = TWM * RPW * ngw;             // at most kRsSzEnt (the plan checks)
  const float rngw = 1.0f / (float)ngw;
  uint32_t stv[SZE], ztv[SZE];
#pragma unroll
  for (int e = 0; e < SZE; ++e) {
    const int idx = lane + 64 * e;
    const int tr = (int)(((float)idx + 0.5f) * rngw);   // idx / ngw (exact: idx, ngw < 2^12)
    const int lr = lrow_of(tr / RPW, tr % RPW);
    const uint32_t off = idx < nent && lr >= 0 ? (uint32_t)((row0 + lr) * p.G + g0 + (idx - tr * ngw)) * 2u : kOob;
    stv[e] = bload2(sr, off);
    ztv[e] = bload2(zr, off);
  }

  // ---- the ring.  Activations by direct-to-LDS loads, coalesced: a step's
  // M x PPR 16-byte pieces (row i, piece p = k/8 within the step) at flat
  // LDS position i*PPR + (p ^ swz), DMA instruction d filling positions
  // 64d .. 64d+63 in lane order; the swizzle XORs the low four bits of p with
  // i*S + p/16, so that the 16 lanes of a fragment read (rows i, K shifts
  // p/16) fall in 16 different bank groups.  Weights in registers. ----
  constexpr int PPR = KSTEP / 8;                 // pieces per activation row and step
  constexpr int NDA = (RPW * PPR + 63) / 64;     // DMA instructions per step (at most)
  auto swz = [&](int i, int pp) { return pp ^ ((i * S + (pp >> 4)) & 15); };
  uint32_t alo[NDA];     // lane part of each DMA instruction's global offset, or kOob
  int akp[NDA];          // the lane's piece within the step (k = 8 * piece)
#pragma unroll
  for (int d = 0; d < NDA; ++d) {
    const int f = 64 * d + lane;
    const int i = f / PPR, pp = swz(i, f - i * PPR);
    akp[d] = pp;
    alo[d] = i < M ? (uint32_t)(i * p.lda) * 2u + 16u * (uint32_t)pp : kOob;
  }
  const int arow_pos = min(r, M - 1) * PPR;      // consumer: flat position of its row
  u4 wv[L][TWM];
  auto aslot = [&](auto slotc) -> u4* {
    constexpr int jj = decltype(slotc)::value;
    return rs_aslot<jj, NW, NJ>()[w];
  };
  // (offsets are pinned in registers before their loads: with a select the
  // compiler would split a load into two branches and lose the load count)
  auto issue = [&](int j, auto slotc) {
    constexpr int jj = decltype(slotc)::value;
    const bool live = j <= je;
    const uint32_t so = live ? (uint32_t)(j * (KSTEP * BPK2 / 2)) : kOobPart;
    u4* const as = aslot(slotc);
#pragma unroll
    for (int d = 0; d < NDA; ++d) {
      uint32_t ao = alo[d] + (uint32_t)(j * KSTEP) * 2u;
      ao = live && j * KSTEP + 8 * akp[d] < p.K ? ao : kOob;
      asm volatile("" : "+v"(ao));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (__attribute__((address_space(3))) void*)(as + 64 * d), 16, ao, 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < TWM; ++t) {
      const int u = j * TW + t;
      const bool in = live && t < TW && u >= u0 && u < u1;
      uint32_t wo = lvo[t] | (in ? 0u : kOobPart);
      asm volatile("" : "+v"(wo));
      wv[jj][t] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo, so, 2));
    }
  };

  f4 acc[TWM];
#pragma unroll
  for (int t = 0; t < TWM; ++t) acc[t] = (f4){0.f, 0.f, 0.f, 0.f};
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u;
  asm volatile("" : "+v"(mlo), "+v"(mhi));  // keep the nibble masks in VGPRs
  const uint32_t magic = 0x64006400u;
  uint32_t* const szw = szt[w];

  // one K step from ring slot jj
  auto consume = [&](int j, auto slotc) {
    constexpr int jj = decltype(slotc)::value;
    const u4* const as = aslot(slotc);
    h8 a[NJ];
#pragma unroll
    for (int q = 0; q < NJ; ++q) {
      const u4 v = as[arow_pos + swz(min(r, M - 1), klane / 8 + q)];
      a[q] = __builtin_bit_cast(h8, perm8_int4(v));
    }
    const int gl = (gsh >= 31 ? 0 : min((j * KSTEP + klane) >> gsh, p.G - 1)) - g0;
#pragma unroll
    for (int t = 0; t < TWM; ++t) {
      const int u = j * TW + t;
      if (t < TW && u >= u0 && u < u1) {   // uniform
        const h2 e = as_h2(szw[(t * RPW + r) * ngw + gl]);
        const h2 s2 = __builtin_shufflevector(e, e, 0, 0), z2 = __builtin_shufflevector(e, e, 1, 1);
        const u4 v = wv[jj][t];
#pragma unroll
        for (int q = 0; q < NJ; ++q) {
          h8 bq;
          if (FMT == FMT_INT4) {
            const uint32_t dw = q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
            bq = dq_int4_dword_perm_r(dw, s2, z2, mlo, mhi, magic);
          } else {
            h2 q0, q1, q2, q3;
            dq_int8_dword(q == 0 ? v.x : v.z, s2, z2, q0, q1);
            dq_int8_dword(q == 0 ? v.y : v.w, s2, z2, q2, q3);
            bq.s01 = q0; bq.s23 = q1; bq.s45 = q2; bq.s67 = q3;
          }
          acc[t] = mfma16x16x32(a[q], bq, acc[t]);
        }
      }
    }
    // the slot's fragments are in registers before its refill is issued
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };

  // ---- stream: L steps in flight.  The scheduling barriers keep each
  // step's loads in issue order, the same on the prologue path as around
  // the loop, so that the load-counter waits stay partial ----
#define SB() __builtin_amdgcn_sched_barrier(0)
  issue(js, std::integral_constant<int, 0>{});
  SB();
  issue(js + 1, std::integral_constant<int, 1>{});
  SB();
  issue(js + 2, std::integral_constant<int, 2>{});
  SB();
  // the scale table, once its loads (issued before the ring) are in
#pragma unroll
  for (int e = 0; e < SZE; ++e) {
    const int idx = lane + 64 * e;
    if (idx < nent) szw[idx] = stv[e] | (ztv[e] << 16);
  }
  SB();
  // (no early exit from the loop body: a step past the wave's last is
  // skipped, its loads read nothing, and every path to the loop head has
  // issued the same loads in the same order)
  for (int jb = js; jb <= je; jb += L) {
    if (jb <= je) consume(jb, std::integral_constant<int, 0>{});
    SB();
    issue(jb + L, std::integral_constant<int, 0>{});
    SB();
    if (jb + 1 <= je) consume(jb + 1, std::integral_constant<int, 1>{});
    SB();
    issue(jb + 1 + L, std::integral_constant<int, 1>{});
    SB();
    if (jb + 2 <= je) consume(jb + 2, std::integral_constant<int, 2>{});
    SB();
    issue(jb + 2 + L, std::integral_constant<int, 2>{});
    SB();
  }
#undef SB
  // the loads past the wave's last step (zeros into the activation slots)
  // land before the slots are reused below
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- fold the K shifts of each tile's accumulator into the wave's
  // partials (both in the wave's own activation slots, free now) ----
  float* const sc = (float*)rs_aslot<0, NW, NJ>()[w];
  float* const part = sc + 256;   // [TWM][M * RPW]
  const int MR = M * RPW;
#pragma unroll
  for (int t = 0; t < TWM; ++t) {
    if (t < TW) {
      mfma_result_fence(acc[t]);
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[(4 * gi + e) * 16 + nl] = acc[t][e];
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      for (int idx = lane; idx < MR; idx += 64) {
        const int i = idx / RPW, rr = idx - i * RPW;
        float v = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) v += sc[(s * RPW + i) * 16 + s * RPW + rr];
        part[t * MR + idx] = v;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  }
  __syncthreads();

  // ---- sum the waves' partials per output (wave order), epilogue ----
  auto tile_sum = [&](int t, int i, int rr) -> float {
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) v += ((const float*)rs_aslot<0, NW, NJ>()[ww])[256 + t * MR + i * RPW + rr];
    return v;
  };
  if (EPI == EPI_SWIGLU) {
    for (int idx = tid; idx < M * valid; idx += NT) {
      const int i = idx / valid, c = idx - i * valid;
      const int t = c / HALF, rr = c - t * HALF;
      const float gv = (float)(_Float16)tile_sum(t, i, rr);
      const float uv = (float)(_Float16)tile_sum(t, i, rr + HALF);
      p.C[(int64_t)i * p.ldc + row0 + c] = (_Float16)(silu_f32(gv) * uv);
    }
  } else {
    for (int idx = tid; idx < M * valid; idx += NT) {
      const int i = idx / valid, lr = idx - i * valid;
      const int t = lr / RPW, rr = lr - t * RPW;
      p.C[(int64_t)i * p.ldc + row0 + lr] = (_Float16)epi_apply(tile_sum(t, i, rr), i, row0 + lr, p.ep);
    }
  }
}

template <int FMT, int EPI, int RPW, int TWM>
hipError_t rs_launch4(const RsArgs& k, int nwg, hipStream_t s) {
  hipLaunchKernelGGL((rstream_kernel<FMT, EPI, RPW, TWM, kRsNW>), dim3(nwg), dim3(64 * kRsNW), 0, s, k);
  return hipGetLastError();
}

template <int FMT, int EPI, int RPW>
hipError_t rs_launch3(const RsArgs& k, const RsPlan& pl, hipStream_t s) {
  switch (pl.twm) {
    case 1: return rs_launch4<FMT, EPI, RPW, 1>(k, pl.nwg, s);
    case 2: return rs_launch4<FMT, EPI, RPW, 2>(k, pl.nwg, s);
    case 4:   // (16-row tiles: at most 2 per workgroup, their partials fill a wave's first slot)
      if constexpr (RPW < 16) return rs_launch4<FMT, EPI, RPW, 4>(k, pl.nwg, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <int FMT, int EPI>
hipError_t rs_launch2(const RsArgs& k, const RsPlan& pl, hipStream_t s) {
  switch (pl.rpw) {
    case 4: return rs_launch3<FMT, EPI, 4>(k, pl, s);
    case 8: return rs_launch3<FMT, EPI, 8>(k, pl, s);
    case 16: return rs_launch3<FMT, EPI, 16>(k, pl, s);
    default: return hipErrorInvalidValue;
  }
}

template <int FMT>
hipError_t rs_launch1(const RsArgs& k, const RsPlan& pl, int epi, hipStream_t s) {
  if (epi == EPI_SWIGLU) return rs_launch2<FMT, EPI_SWIGLU>(k, pl, s);
  return rs_launch2<FMT, EPI_NONE>(k, pl, s);
}

int rs_gshift(const LinearArgs& a) {
  if (a.G == 1) return 31;
  for (int b = 0; b < 31; ++b)
    if (a.g == (1 << b)) return b;
  return -1;
}

}  // namespace

RsPlan rstream_plan(const LinearArgs& a, int num_cus) {
  RsPlan p{};
  p.ok = false;
  if (a.fmt != FMT_INT4) return p;
  if (a.prenorm || a.M < 3 || a.M > 16 || a.K < 1 || (a.K & 7)) return p;
  const int kpl = a.fmt == FMT_INT4 ? 32 : 16;
  if (a.K % (a.fmt == FMT_INT4 ? 2 : 1)) return p;
  if (a.G != 1 && (rs_gshift(a) < 0 || a.g < kpl)) return p;   // a lane's KPL k lie in one group
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return p;
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return p;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return p;
  const int64_t lim = (int64_t)1 << 30;   // offsets stay below the out-of-range part
  if (((int64_t)(a.M - 1) * a.lda + a.K) * 2 >= lim) return p;
  if ((int64_t)a.N * a.G * 2 >= lim) return p;
  const bool swi = a.epi == EPI_SWIGLU;
  const int nrows = swi ? a.F : a.N;
  // tile width: at least M rows and at least 4, at most 4 tiles per
  // workgroup; the least padded work (rows rounded up to whole tiles x K
  // rounded up to whole steps), ties to the narrower tile.  One workgroup
  // per CU: its rows need not fill its last tile.
  int best = 0;
  double best_work = 1e300;
  for (int rpw = 4; rpw <= 16; rpw <<= 1) {
    if (rpw < a.M) continue;
    const int gran = swi ? rpw / 2 : rpw;
    const int R = (nrows + num_cus - 1) / num_cus;
    const int TW = (R + gran - 1) / gran;
    if (TW > 4) continue;
    const int ks = 4 * kpl * (16 / rpw);
    const double work = (double)TW * gran * ((a.K + ks - 1) / ks * ks);
    if (work < best_work) { best_work = work; best = rpw; }
  }
  if (!best) return p;
  const int gran = swi ? best / 2 : best;
  const int R = (nrows + num_cus - 1) / num_cus;   // rows per workgroup; the last tile may be partly empty
  const int TW = (R + gran - 1) / gran;
  const int kstep = 4 * kpl * (16 / best);
  const int KS = (a.K + kstep - 1) / kstep;
  if ((int64_t)(swi ? a.F + R : R) * a.ldw >= lim) return p;
  if ((int64_t)KS * kstep * (a.fmt == FMT_INT4 ? 1 : 2) / 2 >= lim) return p;
  if ((int64_t)TW * KS * kRsNW >= ((int64_t)1 << 31)) return p;
  // tiles the per-wave arrays and scale table are sized for (one tile:
  // the table holds twice the groups, e.g. 14 x 16 rows at K = 18944, M = 16)
  const int twm = TW == 1 ? 1 : TW <= 2 ? 2 : 4;
  if (best == 16 && twm > 2) return p;
  // every wave's scale table (its tile rows x the groups of its K range)
  const int gs = rs_gshift(a);
  const int U = TW * KS;
  for (int w = 0; w < kRsNW; ++w) {
    const int u0 = (w * U) / kRsNW, u1 = ((w + 1) * U) / kRsNW;
    if (u1 <= u0) continue;
    const int js = u0 / TW, je = (u1 - 1) / TW;
    const int ngw = gs >= 31 ? 1 : std::min(((je + 1) * kstep - 1) >> gs, a.G - 1) - ((js * kstep) >> gs) + 1;
    if (twm * best * ngw > kRsSzEnt) return p;
  }
  p.rpw = best;
  p.twm = twm;
  p.R = R;
  p.TW = TW;
  p.KS = KS;
  p.nwg = (nrows + R - 1) / R;
  p.ok = true;
  return p;
}

hipError_t rstream_launch(const LinearArgs& a, const RsPlan& pl, hipStream_t s) {
  if (!pl.ok) return hipErrorInvalidValue;
  RsArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.ep = a.epi_args();
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.K = a.K; k.N = a.N; k.F = a.F; k.G = a.G;
  k.gshift = rs_gshift(a);
  k.R = pl.R; k.TW = pl.TW; k.KS = pl.KS;
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  k.s_bytes = (uint32_t)((int64_t)a.N * a.G * 2);
  k.z_bytes = a.zeros ? k.s_bytes : 0u;
  if (a.fmt != FMT_INT4) return hipErrorInvalidValue;
  return rs_launch1<FMT_INT4>(k, pl, a.epi, s);
}

}  // namespace mq
