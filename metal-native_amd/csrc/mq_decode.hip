// Persistent row-range MFMA GEMV for skinny activations (decode, M <= 16).
//
// Replaces the reference's M<=8 route, dequant_matmul_int{4,8}_vecmat_fp16
// (shaders/matmul_dequant_kernel.metal:229-345, :485-576, dispatched at
// src/ops/matmul.mm:946-1009), and the fp16 vecmat route for B stored [N, K]
// (shaders/matmul_vecmat_kernel.metal:32-139).  Unlike the reference kernel,
// every row of A is computed.
//
// The problem is HBM-bound: the weights are read once and nothing else is
// large.  The kernel is built so that the weight stream starts at once and
// every wave always has D weight loads in flight:
//
//  * Grid: about one workgroup per CU.  Workgroup b owns the contiguous weight
//    rows [b*rows_wg, (b+1)*rows_wg) over the whole of K, so the activations
//    and the rows' scales/zeros are staged into LDS once per CU, not once per
//    handful of rows, and no workgroup ever waits for another.
//  * Work unit: one "step" of one row tile.  The 16 columns of the
//    v_mfma_f32_16x16x32_f16 B operand are RPW weight rows x S = 16/RPW K
//    shifts (column n = row n % RPW at shift n / RPW); a lane reads one
//    16-byte piece, so one wave instruction reads RPW rows x 64*S contiguous
//    bytes (1 KiB).  The A operand holds activation row i at shift s in row
//    s*RPW + i (needs M <= RPW); the result for (activation row i, weight
//    row r) is the sum over s of D[s*RPW + i][s*RPW + r].
//  * The units of a workgroup (tile-major) are cut into NW contiguous ranges,
//    one per wave.  A wave streams its units through a ring of D register
//    slots: slot d is refilled with unit i+D as soon as unit i is consumed.
//    Every load is an unconditional buffer load (lanes past K or past the
//    last row, and refills past the wave's last unit, use an offset outside
//    the buffer, which returns zeros without touching memory), so the
//    compiler's load counter stays exact and a unit waits for its own slot
//    only; barriers wait for LDS traffic only, never for the ring.
//  * The first activation and scale loads are issued before the ring, so
//    staging them into LDS does not wait for the ring either.
//  * When the activations do not fit in LDS, K is cut into chunks (phases)
//    staged in two LDS buffers; the next chunk is loaded into registers during
//    a phase and written to the idle buffer at its end (two barriers per
//    phase).  The weight ring runs across phase boundaries.
//  * Reduction is deterministic: a tile whose units all belong to one wave is
//    added to the LDS accumulator by that wave; a tile shared by consecutive
//    waves is added by the wave holding its first unit, and the others' parts
//    (each wave shares at most its first tile) are added at the phase end in
//    wave order.  fp16 results (and the epilogue) are written at the end.
#include "mq_device.hpp"
#include "mq_launch.hpp"

namespace mq {
namespace {

constexpr int kMaxThreads = 1024;
constexpr int kXpMax = 4;     // activation pieces per thread in a chunk prefetch
constexpr int kXpFirst = 8;   // ... in the first staging batch
constexpr size_t kLdsBudget = 163840;
constexpr uint32_t kOob = 0x80000000u;  // buffer offset outside every range: returns 0

struct DecodeKArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int ldw;
  const _Float16* scales; const _Float16* zeros; const _Float16* bias;
  _Float16* C; int64_t ldc;
  int M, K, G, F, gshift;
  int nrows;      // output rows (N, or F for SwiGLU)
  int rows_wg;    // weight rows per workgroup
  int nsteps;     // K steps per row
  int spc;        // steps per chunk (phase)
  int nchunks;
  int xs_stride;  // LDS activation row stride, halves
  int xp;         // activation pieces per thread per chunk (chunked mode)
  uint32_t a_bytes, sz_bytes, z_bytes;         // buffer extents
  uint32_t off_szs, off_red, off_bnd, off_ws;  // LDS byte offsets
  int sz_chunks;    // 16-byte chunks per staged scale (or zero) region
  uint64_t cpr_m40; // ceil(2^40 / activation pieces per row and chunk)
  uint32_t mlo, mhi, magic;
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u4 bload16_stream(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));  // nt
}
__device__ __forceinline__ u4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// Workgroup barrier that waits for LDS traffic only (the weight loads in
// flight write registers, not memory the other waves read).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// Order this wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// 8 halves of padding after every 128 activations: the K shifts of one wave
// instruction then fall in different LDS banks.
__device__ __forceinline__ int xswz(int k) { return k + ((k >> 7) << 3); }

template <int FMT, int EPI, int RPW, int D, bool CH>
__global__ __launch_bounds__(kMaxThreads) void decode_kernel(DecodeKArgs p) {
  constexpr int S = 16 / RPW;                 // K shifts per MFMA tile
  constexpr int KPL = FmtTraits<FMT>::KPL;    // k per 16-byte piece
  constexpr int KSTEP = 4 * KPL * S;          // k per row per unit
  constexpr int NR = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int BPK2 = (FMT == FMT_INT4) ? 1 : (FMT == FMT_INT8 ? 2 : 4);  // 2 x bytes per k
  extern __shared__ __align__(16) unsigned char smem[];

  const int NT = blockDim.x;
  const int NW = NT >> 6;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nloc = lane & 15, grp = lane >> 4;
  const int rr = nloc % RPW, sh = nloc / RPW;  // weight row in the tile, K shift
  const int M = p.M;
  const int r0 = blockIdx.x * p.rows_wg;
  const int nrw = min(p.rows_wg, p.nrows - r0);
  const int ntiles = (nrw + RPW - 1) / RPW;
  const int KC = p.spc * KSTEP;
  const int XS = p.xs_stride;
  const int xbuf = M * XS;

  _Float16* xs = (_Float16*)smem;                       // [2][M][XS] (one buffer if one phase)
  // scale/zero staging: region (t, r) = tensor t (0 scales, 1 zeros) of weight-row half r holds the
  // 16-byte chunks covering this workgroup's rows [NR][rows_wg][G] entries, starting at the entry
  // delta[r] of the region; a zero chunk follows the regions.
  _Float16* szl = (_Float16*)(smem + p.off_szs);
  float* red = (float*)(smem + p.off_red);              // [NR][rows_wg][M]
  float* bnd = (float*)(smem + p.off_bnd);              // [NW][NR][RPW][M]
  float* wsc = (float*)(smem + p.off_ws) + w * (16 * RPW);  // per wave [16][RPW]
  const int szreg = p.sz_chunks * 8;                 // halves per region
  const int zpad = 2 * NR * szreg;                    // index of the zero chunk

  const rsrc_t wr0 = make_rsrc(p.W + (int64_t)r0 * p.ldw, (uint32_t)nrw * (uint32_t)p.ldw);
  const rsrc_t wr1 = make_rsrc(p.W + ((int64_t)p.F + r0) * p.ldw, NR == 2 ? (uint32_t)nrw * (uint32_t)p.ldw : 0u);
  const rsrc_t ar = make_rsrc(p.A, p.a_bytes);
  const rsrc_t sr = make_rsrc(p.scales, p.sz_bytes);
  const rsrc_t zr = make_rsrc(p.zeros, p.z_bytes);

  auto phase_steps = [&](int c) { return min(p.spc, p.nsteps - c * p.spc); };
  // this wave's unit range [x, y) in phase c
  auto wrange = [&](int c) {
    const int U = ntiles * phase_steps(c);
    return make_int2((w * U) / NW, ((w + 1) * U) / NW);
  };

  // ---- prefetch cursor (wave-uniform): next unit to load ----
  int pc = 0, pt = 0, ps = 0, pleft = 0, pspc = 1;
  auto p_enter = [&](int c) {
    int2 r = make_int2(0, 0);
    while (c < p.nchunks) {
      r = wrange(c);
      if (r.y > r.x) break;
      ++c;
    }
    pc = c;
    pleft = c < p.nchunks ? r.y - r.x : 0;
    pspc = c < p.nchunks ? phase_steps(c) : 1;
    pt = r.x / pspc;
    ps = r.x - pt * pspc;
  };
  auto p_next = [&]() {
    if (--pleft > 0) {
      if (++ps == pspc) { ps = 0; ++pt; }
    } else {
      p_enter(pc + 1);
    }
  };
  // load the unit under the prefetch cursor (zeros once the wave has none left)
  auto wload = [&](u4 (&dst)[NR]) {
    const int rowl = pt * RPW + rr;
    const int k = (pc * p.spc + ps) * KSTEP + sh * 4 * KPL + grp * KPL;
    const bool ok = pleft > 0 && rowl < nrw && k < p.K;
    const uint32_t off = ok ? (uint32_t)(rowl * p.ldw + k * BPK2 / 2) : kOob;
    dst[0] = bload16_stream(wr0, off);
    if (NR == 2) dst[NR - 1] = bload16_stream(wr1, off);
  };

  // ---- activation staging ----
  const int cpr = KC / 8;  // 16-byte activation pieces per row and chunk
  const int xpieces = M * cpr;
  auto row_of = [&](int idx) { return (int)(((uint64_t)(uint32_t)idx * p.cpr_m40) >> 40); };  // idx / cpr
  // skip == true only where no ring load is in flight: a skipped load would
  // otherwise sit younger than ring loads the compiler's counter waits on
  auto x_fetch = [&](int c, int base, u4* v, int cnt, bool skip) {
#pragma unroll
    for (int e = 0; e < cnt; ++e) {
      v[e] = (u4){0u, 0u, 0u, 0u};
      if (!skip || base + w * 64 + e * NT < xpieces) {  // uniform: skip loads with no piece
        const int idx = base + tid + e * NT;
        const int i = row_of(idx), q = idx - i * cpr;
        const int kk = c * KC + 8 * q;
        const bool ok = idx < xpieces && kk < p.K;
        v[e] = bload16(ar, ok ? (uint32_t)((i * p.lda + kk) * 2) : kOob);
      }
    }
  };
  auto x_put = [&](int c, int base, const u4* v, int cnt) {
    _Float16* dst = xs + (c & 1) * xbuf;
#pragma unroll
    for (int e = 0; e < cnt; ++e) {
      const int idx = base + tid + e * NT;
      if (idx < xpieces) {
        const int i = row_of(idx), q = idx - i * cpr;
        u4 vv = v[e];
        if (FMT == FMT_INT4) vv = perm8_int4(vv);
        *(u4*)(dst + i * XS + xswz(8 * q)) = vv;
      }
    }
  };
  // ---- scale/zero staging: raw 16-byte chunks of this workgroup's rows ----
  int delta[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) delta[r] = ((r0 + (r ? p.F : 0)) * p.G) & 7;
  auto s_fetch = [&](u4 (&v)[2 * NR][2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          v[t * NR + r][e] = (u4){0u, 0u, 0u, 0u};
          if (FMT != FMT_F16 && w * 64 + e * NT < p.sz_chunks) {  // uniform
            const int j = tid + e * NT;
            const uint32_t b0 = (uint32_t)(((r0 + (r ? p.F : 0)) * p.G) & ~7) * 2;  // 16-byte aligned
            const uint32_t off = j < p.sz_chunks ? b0 + 16u * j : kOob;
            v[t * NR + r][e] = bload16(t ? zr : sr, off);
          }
        }
  };
  auto s_put = [&](const u4 (&v)[2 * NR][2]) {
#pragma unroll
    for (int q = 0; q < 2 * NR; ++q)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int j = tid + e * NT;
        if (FMT != FMT_F16 && j < p.sz_chunks) *(u4*)(szl + q * szreg + 8 * j) = v[q][e];
      }
  };

  // ---- prologue: first activation/scale batch, then the ring, then LDS ----
  u4 raw[D][NR];
  {
    u4 xf[kXpFirst];
    u4 sv[2 * NR][2];
    x_fetch(0, 0, xf, kXpFirst, true);
    s_fetch(sv);
    p_enter(0);
#pragma unroll
    for (int d = 0; d < D; ++d) {
      wload(raw[d]);
      if (pleft > 0) p_next();
    }
    x_put(0, 0, xf, kXpFirst);
    s_put(sv);
  }
  for (int b = kXpFirst * NT; b < M * cpr; b += kXpFirst * NT) {
    u4 xf[kXpFirst];
    x_fetch(0, b, xf, kXpFirst, false);
    x_put(0, b, xf, kXpFirst);
  }
  if (FMT != FMT_F16 && tid < 8) szl[zpad + tid] = (_Float16)0.f;
  for (int idx = tid; idx < NR * nrw * M; idx += NT) {
    const int r = idx / (nrw * M);
    const int rem = idx - r * nrw * M;
    red[r * p.rows_wg * M + rem] = 0.f;
  }
  lds_barrier();
  u4 xr[kXpMax];
  if (CH) x_fetch(1, 0, xr, kXpMax, false);

  // ---- consume cursor ----
  int total = 0;
  for (int c = 0; c < p.nchunks; ++c) {
    const int2 r = wrange(c);
    total += r.y - r.x;
  }
  int cc = 0, ct = 0, cs = 0, cleft = 0, cspc = 1, cu0 = 0;
  auto c_enter = [&](int c) {
    const int2 r = wrange(c);
    cc = c;
    cspc = phase_steps(c);
    cu0 = r.x;
    ct = r.x / cspc;
    cs = r.x - ct * cspc;
    cleft = r.y - r.x;
  };
  c_enter(0);

  // Tile sums.  Each unit's MFMA chain starts from zero and is added here by
  // VALU right after an explicit result fence, so no path (the flush behind
  // control flow included) ever reads an MFMA destination early.
  f4 acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = (f4){0.f, 0.f, 0.f, 0.f};
  int acc_t = -1;  // tile whose partial sums acc holds

  // add a finished partial tile to the LDS accumulator (or the wave's slot)
  auto put = [&](int t, int r, int row_in_tile, int i, float v) {
    const int rowl = t * RPW + row_in_tile;
    if (rowl >= nrw) return;
    if (t * cspc >= cu0)
      red[(r * p.rows_wg + rowl) * M + i] += v;
    else
      bnd[((w * NR + r) * RPW + row_in_tile) * M + i] = v;
  };
  auto flush = [&](int t) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (RPW == 16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 4 * grp + e;
          if (m < M) put(t, r, nloc, m, acc[r][e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 4 * grp + e;
          if (m / RPW == sh && m % RPW < M) wsc[m * RPW + rr] = acc[r][e];
        }
        wave_lds_sync();
        if (lane < M * RPW) {
          const int i = lane / RPW, rw = lane - i * RPW;
          float v = 0.f;
#pragma unroll
          for (int s = 0; s < S; ++s) v += wsc[(s * RPW + i) * RPW + rw];
          put(t, r, rw, i, v);
        }
        wave_lds_sync();
      }
    }
  };

  auto phase_end = [&](int c) {
    if (CH && c + 1 < p.nchunks) {
      // The next chunk's loads were issued inside this data-dependent control
      // flow; wait for them explicitly rather than trust the derived count.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      x_put(c + 1, 0, xr, kXpMax);
    }
    lds_barrier();
    const int spcc = phase_steps(c);
    const int U = ntiles * spcc;
    for (int idx = tid; idx < NR * nrw * M; idx += NT) {
      const int r = idx / (nrw * M);
      const int rem = idx - r * nrw * M;
      const int rowl = rem / M, i = rem - rowl * M;
      const int t = rowl / RPW, rw = rowl - t * RPW;
      const int wa = ((t * spcc + 1) * NW + U - 1) / U - 1;        // wave holding the tile's first unit
      const int wb = (((t + 1) * spcc) * NW + U - 1) / U - 1;      // ... and its last unit
      if (wa != wb) {
        float v = red[(r * p.rows_wg + rowl) * M + i];
        for (int ww = wa + 1; ww <= wb; ++ww)
          if ((ww * U) / NW < ((ww + 1) * U) / NW) v += bnd[((ww * NR + r) * RPW + rw) * M + i];
        red[(r * p.rows_wg + rowl) * M + i] = v;
      }
    }
    lds_barrier();
    if (CH && c + 2 < p.nchunks) x_fetch(c + 2, 0, xr, kXpMax, false);
  };

  uint32_t mlo = p.mlo, mhi = p.mhi, magic = p.magic;
  asm volatile("" : "+v"(mlo), "+v"(mhi));  // keep the nibble masks resident in VGPRs
  const int xrow = min(rr, M - 1) * XS;
  const int klane = sh * 4 * KPL + grp * KPL;  // this lane's k within a unit

  // consume the unit under the consume cursor from ring slot `slot`
  auto step = [&](const u4 (&slot)[NR]) {
    while (CH && cleft == 0) {  // uniform: the wave's part of phase cc is done
      if (acc_t >= 0) { flush(acc_t); acc_t = -1; }
      phase_end(cc);
      c_enter(cc + 1);
    }
    if (ct != acc_t) {
      if (acc_t >= 0) flush(acc_t);
      acc_t = ct;
#pragma unroll
      for (int r = 0; r < NR; ++r) acc[r] = (f4){0.f, 0.f, 0.f, 0.f};
    }
    const int rowl = ct * RPW + rr;
    const int kin = cs * KSTEP + klane;
    const int k = cc * KC + kin;
    h2 s2[NR], z2[NR];
    if (FMT != FMT_F16) {
      const bool ok = rowl < nrw && k < p.K;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int si = ok ? r * szreg + delta[r] + rowl * p.G + (k >> p.gshift) : zpad;
        const _Float16 sv = szl[si];
        const _Float16 zv = szl[(ok ? NR * szreg : 0) + si];
        s2[r] = (h2){sv, sv};
        z2[r] = (h2){zv, zv};
      }
    }
    const _Float16* xa = xs + (CH ? (cc & 1) * xbuf : 0) + xrow + xswz(kin);
    f4 dacc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) dacc[r] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KPL / 8; ++j) {
      h8 b[NR];
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const u4 v = slot[r];
        if (FMT == FMT_INT4) {
          const uint32_t dw = (j == 0) ? v.x : (j == 1) ? v.y : (j == 2) ? v.z : v.w;
          b[r] = dq_int4_dword_perm_r(dw, s2[r], z2[r], mlo, mhi, magic);
        } else if (FMT == FMT_INT8) {
          const uint32_t d0 = (j == 0) ? v.x : v.z;
          const uint32_t d1 = (j == 0) ? v.y : v.w;
          h2 q0, q1, q2, q3;
          dq_int8_dword(d0, s2[r], z2[r], q0, q1);
          dq_int8_dword(d1, s2[r], z2[r], q2, q3);
          b[r].s01 = q0; b[r].s23 = q1; b[r].s45 = q2; b[r].s67 = q3;
        } else {
          b[r] = __builtin_bit_cast(h8, v);
        }
      }
      const h8 a = *(const h8*)(xa + 8 * j);
#pragma unroll
      for (int r = 0; r < NR; ++r) dacc[r] = mfma16x16x32(a, b[r], dacc[r]);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      mfma_result_fence(dacc[r]);
      acc[r] += dacc[r];
    }
    --cleft;
    if (++cs == cspc) { cs = 0; ++ct; }
  };

  // ---- main loop: whole rounds of the ring, then the tail (no refills) ----
  const int nfull = total - total % D;
  for (int i0 = 0; i0 < nfull; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      step(raw[d]);
      wload(raw[d]);  // unconditional: the load counter stays exact
      if (pleft > 0) p_next();
    }
  }
  const int rem = total - nfull;
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < rem) step(raw[d]);
  if (acc_t >= 0) flush(acc_t);
  for (; cc < p.nchunks; ++cc) phase_end(cc);

  // ---- epilogue: fp16 results of this workgroup's rows ----
  for (int idx = tid; idx < M * nrw; idx += NT) {
    const int i = idx / nrw, rl = idx - i * nrw;
    const int row = r0 + rl;
    if (EPI == EPI_SWIGLU) {
      const float gv = (float)(_Float16)red[rl * M + i];
      const float uv = (float)(_Float16)red[(p.rows_wg + rl) * M + i];
      p.C[(int64_t)i * p.ldc + row] = (_Float16)(silu_f32(gv) * uv);
    } else {
      float v = red[rl * M + i];
      if (EPI == EPI_BIAS) v += (float)p.bias[row];
      p.C[(int64_t)i * p.ldc + row] = (_Float16)v;
    }
  }
}

template <typename KFn>
hipError_t launch_one(KFn fn, bool& attr, const DecodeKArgs& k, const DecodePlan& pl, hipStream_t s) {
  if (!attr && pl.lds_bytes > 65536) {  // raise the dynamic LDS limit once per kernel
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)kLdsBudget);
    if (e != hipSuccess) return e;
    attr = true;
  }
  hipLaunchKernelGGL(fn, dim3(pl.nwg), dim3(64 * pl.nw), pl.lds_bytes, s, k);
  return hipGetLastError();
}

template <int FMT, int EPI, int RPW>
hipError_t launch_rpw(const DecodeKArgs& k, const DecodePlan& pl, hipStream_t s) {
  constexpr int D = (EPI == EPI_SWIGLU) ? 4 : 8;
  static bool attr_ch = false, attr_one = false;
  if (pl.nchunks > 1) return launch_one(decode_kernel<FMT, EPI, RPW, D, true>, attr_ch, k, pl, s);
  return launch_one(decode_kernel<FMT, EPI, RPW, D, false>, attr_one, k, pl, s);
}


template <int FMT, int EPI>
hipError_t launch_epi(const DecodeKArgs& k, const DecodePlan& pl, hipStream_t s) {
  switch (pl.rpw) {
    case 1: return launch_rpw<FMT, EPI, 1>(k, pl, s);
    case 2: return launch_rpw<FMT, EPI, 2>(k, pl, s);
    case 4: return launch_rpw<FMT, EPI, 4>(k, pl, s);
    case 8: return launch_rpw<FMT, EPI, 8>(k, pl, s);
    case 16: return launch_rpw<FMT, EPI, 16>(k, pl, s);
    default: return hipErrorInvalidValue;
  }
}

template <int FMT>
hipError_t launch_fmt(const DecodeKArgs& k, const DecodePlan& pl, int epi, hipStream_t s) {
  if (FMT == FMT_F16 || epi == EPI_NONE) return launch_epi<FMT, EPI_NONE>(k, pl, s);
  if (epi == EPI_BIAS) return launch_epi<FMT, EPI_BIAS>(k, pl, s);
  return launch_epi<FMT, EPI_SWIGLU>(k, pl, s);
}

int kpl_of(int fmt) { return fmt == FMT_INT4 ? 32 : (fmt == FMT_INT8 ? 16 : 8); }
int pow2_ceil(int v) { int r = 1; while (r < v) r <<= 1; return r; }
size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }
int xs_stride_for(int kc) { return ((kc + (kc + 127) / 128 * 8 + 8) + 7) & ~7; }

}  // namespace

bool decode_supported(const LinearArgs& a) {
  const int kpl = kpl_of(a.fmt);
  if (a.M < 1 || a.M > 16) return false;
  if (a.K % kpl != 0) return false;                        // whole 16-byte pieces per row
  if (a.fmt != FMT_F16) {
    if (a.g % kpl != 0 && a.G != 1) return false;          // a piece lies in one group
    if ((a.g & (a.g - 1)) && a.G != 1) return false;       // group index by shift
  }
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  // 32-bit buffer offsets: activations, scales/zeros, and a workgroup's rows
  const int64_t lim = (int64_t)1 << 31;
  if (((int64_t)(a.M - 1) * a.lda + a.K) * 2 >= lim) return false;
  if ((int64_t)a.N * a.G * 2 >= lim || a.ldw >= lim) return false;
  return true;
}

DecodePlan decode_plan(const LinearArgs& a, int num_cus, const DecodeTuning& t) {
  DecodePlan p{};
  const int kpl = kpl_of(a.fmt);
  const int nr = a.epi == EPI_SWIGLU ? 2 : 1;
  const int nrows = a.epi == EPI_SWIGLU ? a.F : a.N;
  const bool quant = a.fmt != FMT_F16;
  // K shifts: as many as M allows, but no wider than K
  int smax = 1;
  while (smax < 16 && 2 * smax * 4 * kpl <= a.K) smax <<= 1;
  int rpw = pow2_ceil(a.M);
  if (rpw < 16 / smax) rpw = 16 / smax;
  if (t.rpw >= rpw && t.rpw <= 16) rpw = t.rpw;
  const int s = 16 / rpw;
  const int kstep = 4 * kpl * s;
  const int nsteps = (a.K + kstep - 1) / kstep;

  const int nwg_target = num_cus * (t.wg_per_cu > 0 ? t.wg_per_cu : 1);
  int rows_wg = (nrows + nwg_target - 1) / nwg_target;
  if (rows_wg < 1) rows_wg = 1;

  auto sz_chunks = [&](int rows) { return (int)(((size_t)rows * a.G * 2 + 15) / 16 + 1); };
  auto fixed_bytes = [&](int rows, int nw) {
    size_t b = quant ? (size_t)(2 * nr * sz_chunks(rows) + 1) * 16 : 0;  // scales/zeros
    b += align16((size_t)nr * rows * a.M * 4);                          // accumulators
    b += align16((size_t)nw * nr * rpw * a.M * 4);                      // shared-tile parts
    if (rpw < 16) b += align16((size_t)nw * 16 * rpw * 4);              // shift sums
    return b;
  };
  while (rows_wg > 1 && fixed_bytes(rows_wg, 16) > kLdsBudget / 2) rows_wg = (rows_wg + 1) / 2;

  int nw = t.max_nw > 0 ? t.max_nw : 16;
  // fewer waves when a workgroup has few units
  const int units = ((rows_wg + rpw - 1) / rpw) * nsteps;
  while (nw > 4 && units < 2 * nw) nw >>= 1;

  const int full_xs = xs_stride_for(nsteps * kstep);
  int spc = nsteps, nchunks = 1, xs_stride = full_xs;
  size_t xbytes = align16((size_t)a.M * full_xs * 2);
  size_t fixed = fixed_bytes(rows_wg, nw);
  if (!t.force_chunks && xbytes + fixed <= kLdsBudget) {
    // whole K in one buffer
  } else {
    if (xbytes + fixed_bytes(rows_wg, 8) <= kLdsBudget && !t.force_chunks && nw > 8) {
      nw = 8;
      fixed = fixed_bytes(rows_wg, nw);
    } else {
      // two chunk buffers; at most kXpMax pieces per thread per chunk
      int spc_max = nsteps;
      while (spc_max > 1) {
        const int kc = spc_max * kstep;
        const size_t xb = 2 * align16((size_t)a.M * xs_stride_for(kc) * 2);
        if (xb + fixed <= kLdsBudget && (size_t)a.M * kc / 8 <= (size_t)kXpMax * 64 * nw &&
            (t.force_chunks == 0 || spc_max <= (nsteps + t.force_chunks - 1) / t.force_chunks))
          break;
        --spc_max;
      }
      nchunks = (nsteps + spc_max - 1) / spc_max;
      spc = (nsteps + nchunks - 1) / nchunks;
      nchunks = (nsteps + spc - 1) / spc;
      xs_stride = xs_stride_for(spc * kstep);
      xbytes = 2 * align16((size_t)a.M * xs_stride * 2);
    }
  }
  p.rpw = rpw;
  p.nw = nw;
  p.rows_wg = rows_wg;
  p.nwg = (nrows + rows_wg - 1) / rows_wg;
  p.nsteps = nsteps;
  p.spc = spc;
  p.nchunks = nchunks;
  p.xs_stride = xs_stride;
  p.xp = (int)(((size_t)a.M * spc * kstep / 8 + 64 * nw - 1) / (64 * nw));
  size_t off = xbytes;
  p.off_szs = (uint32_t)off;
  p.sz_chunks = quant ? sz_chunks(rows_wg) : 0;
  off += quant ? (size_t)(2 * nr * p.sz_chunks + 1) * 16 : 0;
  p.off_red = (uint32_t)off;
  off += align16((size_t)nr * rows_wg * a.M * 4);
  p.off_bnd = (uint32_t)off;
  off += align16((size_t)nw * nr * rpw * a.M * 4);
  p.off_ws = (uint32_t)off;
  if (rpw < 16) off += align16((size_t)nw * 16 * rpw * 4);
  p.lds_bytes = off;
  p.ok = off <= kLdsBudget && (nchunks == 1 || p.xp <= kXpMax) && p.sz_chunks <= 2 * 64 * nw &&
         (int64_t)rows_wg * a.ldw < ((int64_t)1 << 31);
  return p;
}

hipError_t decode_launch(const LinearArgs& a, const DecodePlan& pl, hipStream_t s) {
  if (!pl.ok) return hipErrorInvalidValue;
  DecodeKArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = (int)a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.bias = (const _Float16*)a.bias;
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.K = a.K; k.G = a.G; k.F = a.F;
  k.gshift = 31;  // one group spanning K: index is always 0
  if (a.G != 1)
    for (int b = 0; b < 31; ++b)
      if (a.g == (1 << b)) k.gshift = b;
  k.nrows = a.epi == EPI_SWIGLU ? a.F : a.N;
  k.rows_wg = pl.rows_wg;
  k.nsteps = pl.nsteps;
  k.spc = pl.spc;
  k.nchunks = pl.nchunks;
  k.xs_stride = pl.xs_stride;
  k.xp = pl.xp;
  k.sz_chunks = pl.sz_chunks;
  {
    const uint64_t cpr = (uint64_t)pl.spc * (16 / pl.rpw) * 4 * (a.fmt == FMT_INT4 ? 32 : (a.fmt == FMT_INT8 ? 16 : 8)) / 8;
    k.cpr_m40 = ((1ull << 40) + cpr - 1) / cpr;
  }
  k.off_szs = pl.off_szs; k.off_red = pl.off_red; k.off_bnd = pl.off_bnd; k.off_ws = pl.off_ws;
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  // Buffer loads range-check whole dwords: round the extent up so the dword
  // holding the last entry is readable (an aligned dword never crosses a page;
  // entries past N*G are staged but never used).
  k.sz_bytes = a.fmt == FMT_F16 ? 0u : (uint32_t)(((int64_t)a.N * a.G * 2 + 3) & ~(int64_t)3);
  k.z_bytes = a.zeros ? k.sz_bytes : 0u;
  k.mlo = 0x000F000Fu;
  k.mhi = 0x00F000F0u;
  k.magic = 0x64006400u;
  switch (a.fmt) {
    case FMT_INT4: return launch_fmt<FMT_INT4>(k, pl, a.epi, s);
    case FMT_INT8: return launch_fmt<FMT_INT8>(k, pl, a.epi, s);
    default: return launch_fmt<FMT_F16>(k, pl, a.epi, s);
  }
}

}  // namespace mq
