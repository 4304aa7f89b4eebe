// Split-K MFMA GEMV for skinny activations (decode, M <= 16).
//
// Replaces the reference's M<=8 route, dequant_matmul_int{4,8}_vecmat_fp16
// (shaders/matmul_dequant_kernel.metal:229-345, :485-576, dispatched at
// src/ops/matmul.mm:946-1009), and the fp16 vecmat route for B stored [N, K]
// (shaders/matmul_vecmat_kernel.metal:32-139).  Unlike the reference kernel,
// every row of A is computed.
//
// The problem is HBM-bound (the weights are read once, nothing else is large)
// and, because the dequant of w = half(half(q-8)*s) - z needs two fp16
// roundings per weight, close to VALU-bound as well.  The kernel is built so
// that every CU gets the same number of weight bytes and every weight load is
// in flight from the first instructions on.
//
//  * Row tile: RPW weight rows x S = 16/RPW K shifts form the 16 columns of the
//    B operand of v_mfma_f32_16x16x32_f16.  Column n holds row n % RPW at K
//    shift n / RPW; a lane reads one 16-byte piece, so one wave load covers RPW
//    rows x 64*S contiguous bytes (RPW = 8: whole 128-byte lines).  A row i of
//    the A operand holds activation row i % RPW at shift i / RPW, so the result
//    for (activation i, weight row r) is sum_s D[s*RPW + i][s*RPW + r].  RPW = 8
//    serves M <= 8, RPW = 16 serves M <= 16.
//  * SwiGLU tiles hold RPW/2 gate rows and the matching RPW/2 up rows, so the
//    epilogue has both halves of its output in one wave.
//  * Workgroup = TPW waves = TPW consecutive tiles over one K segment (split).
//    The activations of that segment (re-ordered for the int4 operand layout)
//    and the rows' scales/zeros are staged in LDS once and shared by the waves.
//  * A wave's segment is at most kRing steps, and all of its weight loads are
//    issued before the LDS staging: every byte the wave needs is in flight
//    from its first instructions on.  All loads are unconditional buffer loads
//    (an offset outside the buffer returns zeros without touching memory), so
//    the compiler's load counter is exact and a step waits for its own load.
//  * Splits > 1: each workgroup writes fp32 partials; a per-tile-group counter
//    elects the last arriving workgroup, which sums the partials in split
//    order (deterministic), applies the epilogue, stores fp16 and resets the
//    counter to zero for the next call.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>

namespace mq {
namespace {

constexpr int kRing = 8;      // weight loads in flight per wave
constexpr int kXp = 8;        // activation pieces per thread (staging)
constexpr int kSp = 4;        // scale entries per thread (staging)
constexpr size_t kCntBytes = 65536;  // split-K counters at the start of the workspace

struct GemvKArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros;
  EpiArgs ep;   // element-wise epilogue (kernels without SwiGLU)
  _Float16* C; int64_t ldc;
  int M, K, N, F, G, gshift;
  int T;        // row tiles
  int nq;       // tile groups (workgroups per split)
  int P;        // K splits
  int KS;       // K steps per row (the last split is padded to KK steps with zeros)
  int XS;       // LDS activation row stride (halves)
  int GK;       // LDS scale entries per tile row
  uint32_t off_sz;              // LDS byte offset of the scale table
  uint32_t a_bytes, sz_bytes, z_bytes;
  float* part;                  // [P][M][T*RPW]
  uint32_t* cnt;                // [nq]
};

template <int FMT, int EPI, int RPW, int KK>
__global__ __launch_bounds__(256) void gemv_kernel(GemvKArgs p) {
  constexpr int S = 16 / RPW;
  constexpr int KPL = FmtTraits<FMT>::KPL;       // k per 16-byte piece
  constexpr int KSTEP = 4 * KPL * S;             // k per row per step
  constexpr int NJ = KPL / 8;                    // MFMAs per step
  constexpr int HALF = RPW / 2;
  constexpr int BPK2 = (FMT == FMT_INT4) ? 1 : (FMT == FMT_INT8 ? 2 : 4);  // 2 x bytes per k
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_last;

  const int TPW = blockDim.x >> 6;
  const int NT = blockDim.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = blockIdx.x % p.nq;
  const int split = blockIdx.x / p.nq;
  const int kb = split * KK * KSTEP;
  const int kw = KK * KSTEP;
  const int M = p.M;
  const int t = q * TPW + w;

  _Float16* xs = (_Float16*)smem;                     // [M][XS]
  uint32_t* szl = (uint32_t*)(smem + p.off_sz);       // [TPW*RPW][GK]: s | z << 16

  const int nl = lane & 15, gi = lane >> 4;
  const int r = nl % RPW, sh = nl / RPW;              // weight row in tile, K shift
  const int klane = sh * 4 * KPL + gi * KPL;          // this lane's k within a step

  // ---- weight buffer of this wave's tile ----
  // plain: rows [t*RPW, t*RPW + RPW); SwiGLU: gate rows [t*HALF, +HALF) and up
  // rows F + the same.  Rows past the end read as zeros (outside the range).
  uint32_t rows_span;
  const unsigned char* wbase;
  uint32_t roff;
  if (EPI == EPI_SWIGLU) {
    const int f0 = t * HALF;
    wbase = p.W + (int64_t)f0 * p.ldw;
    const int valid = max(0, min(HALF, p.F - f0));
    rows_span = (uint32_t)((p.F + valid) * p.ldw);
    // gate rows f0+r (r < HALF), up rows F+f0+(r-HALF); gate rows past F would
    // land in the up region, so they are sent outside the range instead.
    const bool ok = (r < HALF) ? (r < valid) : (r - HALF < valid);
    roff = ok ? (uint32_t)(((r < HALF) ? r : p.F + r - HALF) * p.ldw) : kOob;
  } else {
    const int r0 = t * RPW;
    wbase = p.W + (int64_t)r0 * p.ldw;
    const int valid = max(0, min(RPW, p.N - r0));
    rows_span = (uint32_t)(valid * p.ldw);
    roff = (uint32_t)(r * p.ldw);
  }
  // the tile is wave-uniform; say so, or the loads become waterfall loops
  {
    const uint64_t b = (uint64_t)wbase;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    wbase = (const unsigned char*)(((uint64_t)hi << 32) | lo);
    rows_span = __builtin_amdgcn_readfirstlane(rows_span);
  }
  const rsrc_t wr = make_rsrc(wbase, rows_span);
  auto wload = [&](int jl) -> u4 {
    const int k = kb + jl * KSTEP + klane;
    const uint32_t off = (k < p.K && roff != kOob) ? roff + (uint32_t)(k * BPK2 / 2) : kOob;
    return bload16_nt(wr, off);
  };

  // ---- staging loads: activations of the segment, then scales/zeros ----
  const rsrc_t ar = make_rsrc(p.A, p.a_bytes);
  const int ppr = kw >> 3;              // 16-byte activation pieces per row
  const int npieces = M * ppr;
  u4 xv[kXp];
#pragma unroll
  for (int e = 0; e < kXp; ++e) {
    const int idx = tid + e * NT;
    const int i = idx / ppr, c = idx - i * ppr;
    const int k = kb + 8 * c;
    const bool ok = idx < npieces && k < p.K;
    xv[e] = bload16(ar, ok ? (uint32_t)((i * p.lda + k) * 2) : kOob);
  }
  const int g0 = kb >> p.gshift;
  const int GK = p.GK;
  const int nsz = TPW * RPW * GK;
  uint32_t sv[kSp], zv[kSp];
  if (FMT != FMT_F16) {
    const rsrc_t sr = make_rsrc(p.scales, p.sz_bytes);
    const rsrc_t zr = make_rsrc(p.zeros, p.z_bytes);
#pragma unroll
    for (int e = 0; e < kSp; ++e) {
      const int idx = tid + e * NT;
      const int row = idx / GK, gg = idx - row * GK;
      const int tw = q * TPW + row / RPW, rr = row % RPW;
      int grow;
      bool ok;
      if (EPI == EPI_SWIGLU) {
        const int f = tw * HALF + rr % HALF;
        ok = f < p.F;
        grow = rr < HALF ? f : p.F + f;
      } else {
        grow = tw * RPW + rr;
        ok = grow < p.N;
      }
      ok = ok && idx < nsz && g0 + gg < p.G;
      const uint32_t off = ok ? (uint32_t)((grow * p.G + g0 + gg) * 2) : kOob;
      sv[e] = bload2(sr, off);
      zv[e] = bload2(zr, off);
    }
  }

  // ---- the weight ring ----
  u4 raw[KK];
#pragma unroll
  for (int d = 0; d < KK; ++d) raw[d] = wload(d);

  // ---- LDS staging (waits for the staging loads only) ----
#pragma unroll
  for (int e = 0; e < kXp; ++e) {
    const int idx = tid + e * NT;
    if (idx < npieces) {
      const int i = idx / ppr, c = idx - i * ppr;
      u4 v = xv[e];
      if (FMT == FMT_INT4) v = perm8_int4(v);
      *(u4*)(xs + i * p.XS + xswz(8 * c)) = v;
    }
  }
  if (FMT != FMT_F16) {
#pragma unroll
    for (int e = 0; e < kSp; ++e) {
      const int idx = tid + e * NT;
      if (idx < nsz) szl[idx] = (sv[e] & 0xffffu) | (zv[e] << 16);
    }
  }
  __syncthreads();

  // ---- consume ----
  const int xrow = min(r, M - 1) * p.XS;
  const uint32_t* szrow = szl + (w * RPW + r) * GK;
  f4 acc = (f4){0.f, 0.f, 0.f, 0.f};
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u;
  asm volatile("" : "+v"(mlo), "+v"(mhi));  // keep the nibble masks in VGPRs
  const uint32_t magic = 0x64006400u;

  auto step = [&](const u4 v, int jl) {
    const int kin = jl * KSTEP + klane;
    h2 s2 = (h2){(_Float16)0.f, (_Float16)0.f}, z2 = s2;
    if (FMT != FMT_F16) {
      // broadcast halves: the packed ops' operand selectors read them in place
      const h2 e = as_h2(szrow[((kb + kin) >> p.gshift) - g0]);
      s2 = __builtin_shufflevector(e, e, 0, 0);
      z2 = __builtin_shufflevector(e, e, 1, 1);
    }
    const _Float16* xa = xs + xrow + xswz(kin);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      h8 b;
      if (FMT == FMT_INT4) {
        const uint32_t dw = (j == 0) ? v.x : (j == 1) ? v.y : (j == 2) ? v.z : v.w;
        b = dq_int4_dword_perm_r(dw, s2, z2, mlo, mhi, magic);
      } else if (FMT == FMT_INT8) {
        const uint32_t d0 = (j == 0) ? v.x : v.z;
        const uint32_t d1 = (j == 0) ? v.y : v.w;
        h2 q0, q1, q2, q3;
        dq_int8_dword(d0, s2, z2, q0, q1);
        dq_int8_dword(d1, s2, z2, q2, q3);
        b.s01 = q0; b.s23 = q1; b.s45 = q2; b.s67 = q3;
      } else {
        // k past K reads zeros from the buffer, so no select is needed
        b = __builtin_bit_cast(h8, v);
      }
      const h8 a = *(const h8*)(xa + 8 * j);
      acc = mfma16x16x32(a, b, acc);
    }
  };

#pragma unroll
  for (int d = 0; d < KK; ++d) step(raw[d], d);
  mfma_result_fence(acc);

  // ---- combine the K shifts: holder lanes get out(i = 4*gi + e, row r) ----
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = acc[e];
    if (S == 2) v[e] += __shfl(v[e], (lane + 40) & 63);
  }
  const bool holder = (S == 2) ? (gi < 2 && nl < 8) : true;

  if (p.P == 1) {
    if (EPI == EPI_SWIGLU) {
      float u[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) u[e] = __shfl(v[e], (lane + HALF) & 63);
      const int f = t * HALF + r;
      if (holder && r < HALF && f < p.F) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * gi + e;
          if (i < M) {
            const float gv = (float)(_Float16)v[e];
            const float uv = (float)(_Float16)u[e];
            p.C[(int64_t)i * p.ldc + f] = (_Float16)(silu_f32(gv) * uv);
          }
        }
      }
    } else {
      const int row = t * RPW + r;
      if (holder && row < p.N) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * gi + e;
          if (i < M) p.C[(int64_t)i * p.ldc + row] = (_Float16)epi_apply(v[e], i, row, p.ep);
        }
      }
    }
    return;
  }

  // ---- split-K: partials, last-arriver reduction ----
  // Ordering: every access to the partials is a system-scope atomic (stores
  // written through to memory, loads served from memory), and a workgroup's
  // stores are acknowledged (s_waitcnt vmcnt(0)) before its counter
  // increment.  That is the gfx942/gfx950 lowering of a system-scope release
  // (and, on the reading side, acquire) minus the L2 writeback/invalidate,
  // which exist only to publish non-atomic accesses; none are made here.
  // The last workgroup to arrive sums the partials in split order; no
  // workgroup ever waits for another.
  const int NP = p.T * RPW;
  if (holder && t < p.T) {  // tiles past T (last group) have no partial slots
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 4 * gi + e;
      if (i < M)
        __hip_atomic_store(p.part + ((int64_t)split * M + i) * NP + t * RPW + r, v[e], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(p.cnt + q, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    s_last = prev == (uint32_t)(p.P - 1);
  }
  __syncthreads();
  if (!s_last) return;
  const int64_t pstride = (int64_t)M * NP;
  if (EPI == EPI_SWIGLU) {
    const int nout = TPW * HALF;
    for (int idx = tid; idx < M * nout; idx += NT) {
      const int i = idx / nout, c = idx - i * nout;
      const int tl = c / HALF, fr = c - tl * HALF;
      const int tt = q * TPW + tl;
      const int f = tt * HALF + fr;
      if (tt >= p.T || f >= p.F) continue;
      const float* src = p.part + (int64_t)i * NP + tt * RPW + fr;
      float gs = 0.f, us = 0.f;
      for (int sp = 0; sp < p.P; ++sp) {
        gs += ld_coherent(src + sp * pstride);
        us += ld_coherent(src + sp * pstride + HALF);
      }
      const float gv = (float)(_Float16)gs;
      const float uv = (float)(_Float16)us;
      p.C[(int64_t)i * p.ldc + f] = (_Float16)(silu_f32(gv) * uv);
    }
  } else {
    const int nout = TPW * RPW;
    for (int idx = tid; idx < M * nout; idx += NT) {
      const int i = idx / nout, c = idx - i * nout;
      const int row = q * nout + c;
      if (row >= p.N) continue;
      const float* src = p.part + (int64_t)i * NP + row;
      float s = 0.f;
      for (int sp = 0; sp < p.P; ++sp) s += ld_coherent(src + sp * pstride);
      p.C[(int64_t)i * p.ldc + row] = (_Float16)epi_apply(s, i, row, p.ep);
    }
  }
  if (tid == 0) __hip_atomic_store(p.cnt + q, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

template <int FMT, int EPI, int RPW, int KK>
hipError_t launch4(const GemvKArgs& k, const GemvPlan& pl, hipStream_t s) {
  auto fn = gemv_kernel<FMT, EPI, RPW, KK>;
  if (pl.lds_bytes > 65536) {
    hipError_t e = allow_dynamic_lds((const void*)fn, 163840);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3(pl.nwg), dim3(64 * pl.tpw), pl.lds_bytes, s, k);
  return hipGetLastError();
}

template <int FMT, int EPI, int RPW>
hipError_t launch3(const GemvKArgs& k, const GemvPlan& pl, hipStream_t s) {
  switch (pl.kk) {
    case 1: return launch4<FMT, EPI, RPW, 1>(k, pl, s);
    case 2: return launch4<FMT, EPI, RPW, 2>(k, pl, s);
    case 3: return launch4<FMT, EPI, RPW, 3>(k, pl, s);
    case 4: return launch4<FMT, EPI, RPW, 4>(k, pl, s);
    case 5: return launch4<FMT, EPI, RPW, 5>(k, pl, s);
    case 6: return launch4<FMT, EPI, RPW, 6>(k, pl, s);
    case 7: return launch4<FMT, EPI, RPW, 7>(k, pl, s);
    case 8: return launch4<FMT, EPI, RPW, 8>(k, pl, s);
    default: return hipErrorInvalidValue;
  }
}

template <int FMT, int EPI>
hipError_t launch2(const GemvKArgs& k, const GemvPlan& pl, hipStream_t s) {
  return pl.rpw == 8 ? launch3<FMT, EPI, 8>(k, pl, s) : launch3<FMT, EPI, 16>(k, pl, s);
}

template <int FMT>
hipError_t launch1(const GemvKArgs& k, const GemvPlan& pl, int epi, hipStream_t s) {
  if (FMT == FMT_F16 || epi != EPI_SWIGLU) return launch2<FMT, EPI_NONE>(k, pl, s);
  return launch2<FMT, EPI_SWIGLU>(k, pl, s);
}

int xswz_host(int k) { return k + ((k >> 7) << 3); }
int kpl_of(int fmt) { return fmt == FMT_INT4 ? 32 : (fmt == FMT_INT8 ? 16 : 8); }
size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }
int gshift_of(const LinearArgs& a) {
  if (a.fmt == FMT_F16 || a.G == 1) return 31;
  for (int b = 0; b < 31; ++b)
    if (a.g == (1 << b)) return b;
  return -1;
}

}  // namespace

bool gemv_supported(const LinearArgs& a) {
  const int kpl = kpl_of(a.fmt);
  if (a.M < 1 || a.M > 16) return false;
  if (a.K % kpl != 0) return false;                    // whole 16-byte pieces per row
  if (a.fmt != FMT_F16 && a.G != 1 && (gshift_of(a) < 0 || a.g < kpl)) return false;
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  const int64_t lim = (int64_t)1 << 31;
  if (((int64_t)(a.M - 1) * a.lda + a.K) * 2 >= lim) return false;
  if ((int64_t)a.N * a.G * 2 >= lim) return false;
  if ((int64_t)(a.epi == EPI_SWIGLU ? a.F + 16 : 16) * a.ldw >= lim) return false;
  return true;
}

GemvPlan gemv_plan(const LinearArgs& a, int num_cus, const GemvTuning& tu) {
  GemvPlan p{};
  const int kpl = kpl_of(a.fmt);
  const int rpw = a.M <= 8 ? 8 : 16;
  const int S = 16 / rpw;
  const int kstep = 4 * kpl * S;
  const int KS = (a.K + kstep - 1) / kstep;
  const int T = a.epi == EPI_SWIGLU ? (a.F + rpw / 2 - 1) / (rpw / 2) : (a.N + rpw - 1) / rpw;
  const bool quant = a.fmt != FMT_F16;
  const int gsh = gshift_of(a);
  const size_t row_bytes = (size_t)kstep * (a.fmt == FMT_INT4 ? 1 : (a.fmt == FMT_INT8 ? 2 : 4)) / 2;
  const double step_bytes = (double)rpw * row_bytes;  // weight bytes per wave step

  double best = 1e300;
  for (int tpw = 1; tpw <= 4; tpw <<= 1) {
    if (tu.tpw && tpw != tu.tpw) continue;
    const int nq = (T + tpw - 1) / tpw;
    const int nt = 64 * tpw;
    for (int KKmax = 1; KKmax <= kRing; ++KKmax) {
      const int P = (KS + KKmax - 1) / KKmax;
      if (P > 4096) continue;
      if (tu.steps && KKmax != tu.steps) continue;
      const int kw = KKmax * kstep;
      // staging capacity
      if ((int64_t)a.M * kw / 8 > (int64_t)kXp * nt) continue;
      int GK = 1;
      if (quant && a.G > 1) GK = ((kw - 1) >> gsh) + 2;  // window may straddle one extra group
      if (quant && (int64_t)tpw * rpw * GK > (int64_t)kSp * nt) continue;
      const size_t xs_stride = (size_t)((xswz_host(kw) + 8 + 7) & ~7);
      const size_t lds = align16((size_t)a.M * xs_stride * 2) + (quant ? (size_t)tpw * rpw * GK * 4 : 0);
      if (lds > 65536) continue;
      const int64_t nwg = (int64_t)nq * P;
      if (nwg > 0x7fffffff) continue;
      // Time model (microseconds) for the most loaded CU: weight streaming at
      // its share of ~7 TB/s or the dequant VALU at 64 lane-ops per clock,
      // plus a fixed cost per resident wave (staging the activation window
      // and scales, the partial store: about 0.25 us each, measured at the
      // config-2 shapes), plus the split-K partial traffic.
      const double wg_cu = std::ceil((double)nwg / num_cus);
      const double bytes_cu = wg_cu * tpw * KKmax * step_bytes;
      const double t_mem = bytes_cu / 27.0e3;
      const double wpb = a.fmt == FMT_INT4 ? 2.0 : 1.0;                      // weights per byte
      const double ops = a.fmt == FMT_INT4 ? 2.2 : (a.fmt == FMT_INT8 ? 2.0 : 0.3);
      const double t_valu = bytes_cu * wpb * ops / (64.0 * 2400.0);
      const double t_wave = 0.25 * wg_cu * tpw;
      const double t_part = P > 1 ? (double)P * a.M * T * rpw * 8.0 / num_cus / 27.0e3 : 0.0;
      const double cost = std::max(t_mem, t_valu) + t_wave + t_part;
      if (cost < best * 0.999) {
        best = cost;
        p.rpw = rpw; p.tpw = tpw; p.P = P; p.kk = KKmax; p.nq = nq; p.nwg = (int)nwg;
        p.KS = KS; p.T = T; p.GK = GK; p.XS = (int)xs_stride;
        p.off_sz = (uint32_t)align16((size_t)a.M * xs_stride * 2);
        p.lds_bytes = lds;
      }
    }
  }
  p.ok = best < 1e299;
  p.ws_bytes = 0;
  if (p.ok && p.P > 1) {
    // The counter region has one fixed size for every shape: counters of one
    // call must never sit where another call's partial sums were written.
    p.cnt_bytes = kCntBytes;
    if ((size_t)p.nq * 4 > kCntBytes) p.ok = false;
    p.ws_bytes = p.cnt_bytes + (size_t)p.P * a.M * p.T * p.rpw * 4;
  }
  return p;
}

// ---- fixed scratch (mq_dequant_matmul_noalloc) ----
// Device memory of the split-K counters and partials for callers that cannot
// allocate.  In host code `scratch` names a host-side stand-in, not a device
// address: every use goes through the per-device address from
// hipGetSymbolAddress.  Calls that overlap on one GPU share it and race.
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void clear_words_kernel(uint32_t* p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

size_t gemv_scratch_bytes() { return kScratchBytes; }

hipError_t gemv_scratch(hipStream_t s, void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    // the counters start at zero (every launch leaves them zero again); a
    // fill kernel, not a memset, so that a capturing caller records a kernel
    hipLaunchKernelGGL(clear_words_kernel, dim3(64), dim3(256), 0, s, (uint32_t*)p, (int)(kCntBytes / 4));
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    addr[dev] = p;
  }
  *out = addr[dev];
  return hipSuccess;
}

hipError_t gemv_launch(const LinearArgs& a, const GemvPlan& pl, void* ws, hipStream_t s) {
  if (!pl.ok) return hipErrorInvalidValue;
  GemvKArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.ep = a.epi_args();
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.K = a.K; k.N = a.N; k.F = a.F; k.G = a.G;
  k.gshift = gshift_of(a);
  k.T = pl.T; k.nq = pl.nq; k.P = pl.P; k.KS = pl.KS; k.XS = pl.XS; k.GK = pl.GK;
  k.off_sz = pl.off_sz;
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  // buffer loads range-check whole dwords: round up so the dword holding the
  // last entry is readable
  k.sz_bytes = a.fmt == FMT_F16 ? 0u : (uint32_t)(((int64_t)a.N * a.G * 2 + 3) & ~(int64_t)3);
  k.z_bytes = a.zeros ? k.sz_bytes : 0u;
  if (pl.P > 1) {
    if (!ws) return hipErrorInvalidValue;
    k.cnt = (uint32_t*)ws;
    k.part = (float*)((char*)ws + pl.cnt_bytes);
  }
  switch (a.fmt) {
    case FMT_INT4: return launch1<FMT_INT4>(k, pl, a.epi, s);
    case FMT_INT8: return launch1<FMT_INT8>(k, pl, a.epi, s);
    default: return launch1<FMT_F16>(k, pl, a.epi, s);
  }
}

}  // namespace mq
