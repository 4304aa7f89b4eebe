// Row-block MFMA GEMV for skinny activations (decode, M <= 64).
//
// Replaces the reference's M<=8 route, dequant_matmul_int{4,8}_vecmat_fp16
// (shaders/matmul_dequant_kernel.metal:229-345, :485-576, dispatched at
// src/ops/matmul.mm:946-1009), and the fp16 vecmat route for B stored [N, K]
// (shaders/matmul_vecmat_kernel.metal:32-139).  Unlike the reference kernel,
// every row of A is computed.
//
// One workgroup owns 16 weight rows (for SwiGLU: 16 gate rows and the
// matching 16 up rows) over the whole of K, so no workgroup ever waits for
// another and no workspace is needed.  Its NW wavefronts split K: in chunk c,
// wave w handles K step c*NW + w, where a step is one 16-byte piece of each of
// the 16 rows per lane group (lane l: row l & 15, piece l >> 4), i.e. 16 rows
// x 64 contiguous bytes per wave.  Consecutive waves therefore sweep each row
// contiguously.
//   * Weights stream through a ring of D register slots per lane: the loads of
//     step i+D are issued as soon as step i has been consumed, so D steps of
//     every wave are always in flight.
//   * The activation chunk of the next step is loaded into registers while the
//     current one is consumed from LDS (two LDS buffers, one barrier per step);
//     int4 activations are stored in the MFMA operand order of the cheap
//     nibble extraction.
//   * Each 16-byte weight piece is dequantized in registers into the B operand
//     of v_mfma_f32_16x16x32_f16 (fp16 products, fp32 accumulation); rows of
//     A beyond M are zero.
//   * The NW partial tiles are summed in LDS in wave order (deterministic),
//     then the epilogue runs and fp16 results are stored.
#include "mq_device.hpp"
#include "mq_launch.hpp"

namespace mq {
namespace {

struct GemvKArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros; const _Float16* bias;
  _Float16* C; int64_t ldc;
  int M, N, K, g, G, F, gshift;
  int nchunks;  // chunked mode: K chunks
  int nsteps;   // K steps (KSTEP each)
  int kpad;     // whole-K mode: K rounded up to whole steps
  uint32_t mlo, mhi, magic;  // nibble masks and the fp16 1024.0 pair (kept out of immediates)
  int xs_stride;  // whole-K kernel: LDS activation row stride (halves)
  uint64_t gp_m64;  // whole-K kernel: ceil(2^40 / (G+1)); x / (G+1) = (x * gp_m64) >> 40 for x < 2^24
};

__device__ __forceinline__ u4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load((const u4*)p);
}

// Sum the NW wave tiles in LDS (in wave order, so results do not depend on
// scheduling), apply the epilogue and store fp16.  Lane l of a wave holds
// D[m = 16*mb + 4*(l>>4) + e][col = l & 15] of its 16-column tile.
template <int NW, int NR, int MB, int EPI>
__device__ __forceinline__ void gemv_reduce_store(const GemvKArgs& p, f4 (&acc)[NR][MB], unsigned char* smem,
                                                  int tid, int w, int nloc, int grp) {
  constexpr int NT = 64 * NW;
  float* red = (float*)smem;  // [NW][NR][M][16]
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * mb + 4 * grp + e;
        if (m < p.M) red[((w * NR + r) * p.M + m) * 16 + nloc] = acc[r][mb][e];
      }
  __syncthreads();
  for (int idx = tid; idx < p.M * 16; idx += NT) {
    const int m = idx >> 4, c = idx & 15;
    const int row = 16 * blockIdx.x + c;
    float s[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      s[r] = 0.f;
      for (int ww = 0; ww < NW; ++ww) s[r] += red[((ww * NR + r) * p.M + m) * 16 + c];
    }
    if (EPI == EPI_SWIGLU) {
      if (row < p.F) {
        const float gv = (float)(_Float16)s[0];
        const float uv = (float)(_Float16)s[NR - 1];
        p.C[(int64_t)m * p.ldc + row] = (_Float16)(silu_f32(gv) * uv);
      }
    } else if (row < p.N) {
      float v = s[0];
      if (EPI == EPI_BIAS) v += (float)p.bias[row];
      p.C[(int64_t)m * p.ldc + row] = (_Float16)v;
    }
  }
}

// Whole-K kernel: the activations (all of K) and the per-group scales/zeros
// of the workgroup's rows are staged in LDS once; the main loop then has no
// barrier and waits only for the oldest weight load of the ring.
// Rows past N are clamped to a valid row (their output columns are never
// stored); A rows past M are clamped to row M-1 (they only feed output rows
// that are never stored); steps past K (only in the last step when
// K % KSTEP != 0) have their weights zeroed, and A is zero there.
// Whole-K kernel.
//
// One workgroup owns RPW weight rows (RPW in {2, 4, 8, 16}) over the whole
// of K; its NW waves take the K steps round-robin (wave w: steps w, w+NW, ...).
// The 16 columns of the MFMA tile are RPW weight rows x S = 16/RPW K shifts:
// column n holds row n % RPW at shift n / RPW, i.e. the lane's 16-byte piece
// sits 64*(n / RPW) bytes further along the row, so one wave instruction reads
// RPW rows x 64*S contiguous bytes.  A row m holds activation row m % RPW at
// the same shift m / RPW (needs M <= RPW); the result for (activation row i,
// weight row r) is the sum over shifts s of D[s*RPW + i][s*RPW + r].
//
// The loop body has no branches on lane data: weights stream through a ring
// of D register slots, refilled while steps remain (a wave-uniform branch);
// lanes past K in the last step read
// their row's last piece and take scale = zero = 0 from a zero pad entry of
// the LDS scale table, with zero activations there, so they add exactly 0.
// The activations (swizzled: 8 halves of padding after every 128 so that the
// K shifts fall in different LDS banks) and the scales/zeros are loaded before
// the ring so that waiting for them never waits for HBM.
__device__ __forceinline__ int xswz(int k) { return k + ((k >> 7) << 3); }

template <int FMT, int NW, int RPW, int EPI, int D>
__global__ __launch_bounds__(64 * NW) void gemv_full_kernel(GemvKArgs p) {
  constexpr int S = 16 / RPW;                      // K shifts per MFMA tile
  constexpr int KPL = FmtTraits<FMT>::KPL;
  constexpr int KSTEP = 4 * KPL * S;               // k per row per wave step
  constexpr int NR = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int NT = 64 * NW;
  constexpr int BPK2 = (FMT == FMT_INT4) ? 1 : (FMT == FMT_INT8 ? 2 : 4);  // 2 x bytes per k
  constexpr int XPB = 4;                          // activation pieces per thread per batch
  constexpr int SPB = 4;                          // scale/zero entries per thread per batch
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nloc = lane & 15, grp = lane >> 4;
  const int rr = nloc % RPW, sh = nloc / RPW;      // weight row in the block, K shift
  const int nrows = (EPI == EPI_SWIGLU) ? p.F : p.N;
  const int row0 = RPW * blockIdx.x;

  // LDS: activations [M][XS] (swizzled) | scales/zeros [NR*RPW][G+1] | partial tiles
  const int XS = p.xs_stride;
  _Float16* xs = (_Float16*)smem;
  uint32_t* szs = (uint32_t*)(smem + (size_t)p.M * XS * 2);
  const int GP = p.G + 1;                          // + one zero entry for lanes past K

  const int kl = sh * 4 * KPL + grp * KPL;         // this lane's k within a step
  const int nsw = (p.nsteps - w + NW - 1) / NW;    // this wave's steps

  // ---- prologue ----
  const int prow = p.kpad / 8;                     // 16-byte activation pieces per row
  const int xbr = (prow + NT * XPB - 1) / (NT * XPB);
  const int xbt = p.M * xbr;                       // activation batches
  auto x_load = [&](int bt, u4 (&v)[XPB]) {
    const int m = bt / xbr, c0 = (bt - m * xbr) * NT * XPB;  // uniform
#pragma unroll
    for (int e = 0; e < XPB; ++e) {
      const int c = c0 + tid + e * NT;
      v[e] = (u4){0u, 0u, 0u, 0u};
      if (c < prow && 8 * c < p.K) v[e] = *(const u4*)(p.A + (int64_t)m * p.lda + 8 * c);
    }
  };
  auto x_store = [&](int bt, u4 (&v)[XPB]) {
    const int m = bt / xbr, c0 = (bt - m * xbr) * NT * XPB;
#pragma unroll
    for (int e = 0; e < XPB; ++e) {
      const int c = c0 + tid + e * NT;
      if (c < prow) {
        u4 vv = v[e];
        if (FMT == FMT_INT4) vv = perm8_int4(vv);
        *(u4*)(xs + m * XS + xswz(8 * c)) = vv;
      }
    }
  };
  const int stot = (FMT != FMT_F16) ? NR * RPW * GP : 0;
  auto s_load = [&](int b0, uint32_t (&v)[SPB]) {
#pragma unroll
    for (int e = 0; e < SPB; ++e) {
      const int idx = b0 + tid + e * NT;
      v[e] = 0u;
      if (idx < stot) {
        const int lr = (int)(((uint64_t)(uint32_t)idx * p.gp_m64) >> 40);  // idx / GP, exact
        const int gi = idx - lr * GP;
        if (gi < p.G) {
          const int r = lr / RPW, ri = lr - r * RPW;
          const int64_t at = (int64_t)(min(row0 + ri, nrows - 1) + (r ? p.F : 0)) * p.G + gi;
          const uint32_t sv = __builtin_bit_cast(uint16_t, p.scales[at]);
          const uint32_t zv = p.zeros ? __builtin_bit_cast(uint16_t, p.zeros[at]) : 0u;
          v[e] = sv | (zv << 16);
        }
      }
    }
  };
  for (int bt = 0; bt + 1 < xbt; ++bt) {  // all but the last activation batch
    u4 v[XPB];
    x_load(bt, v);
    x_store(bt, v);
  }
  int sb0 = 0;
  for (; sb0 + NT * SPB < stot; sb0 += NT * SPB) {  // all but the last scale batch
    uint32_t v[SPB];
    s_load(sb0, v);
#pragma unroll
    for (int e = 0; e < SPB; ++e)
      if (sb0 + tid + e * NT < stot) szs[sb0 + tid + e * NT] = v[e];
  }
  u4 xv[XPB];
  uint32_t sv[SPB];
  x_load(xbt - 1, xv);
  s_load(sb0, sv);

  // ---- weight ring ----
  const unsigned char* wrow[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int row = min(row0 + rr, nrows - 1) + (r ? p.F : 0);  // rows past N: never stored
    wrow[r] = p.W + (int64_t)row * p.ldw;
  }
  const int klast = p.K - KPL;                     // last in-range piece of a row
  u4 raw[D][NR];
  auto wload = [&](int i, int slot) {
    // uniform: refills past the wave's last step repeat it; a wave without
    // steps (nsw == 0) reads step w, clamped into the row like any other
    const int ic = max(min(i, nsw - 1), 0);
    const int k = min((ic * NW + w) * KSTEP + kl, klast);
#pragma unroll
    for (int r = 0; r < NR; ++r) raw[slot][r] = ld16_stream(wrow[r] + (int64_t)k * BPK2 / 2);
  };
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < nsw) wload(d, d);
  x_store(xbt - 1, xv);
#pragma unroll
  for (int e = 0; e < SPB; ++e)
    if (sb0 + tid + e * NT < stot) szs[sb0 + tid + e * NT] = sv[e];
  __syncthreads();

  // ---- main loop ----
  uint32_t mlo = p.mlo, mhi = p.mhi, magic = p.magic;
  asm volatile("" : "+v"(mlo), "+v"(mhi));  // keep the masks resident in VGPRs
  const _Float16* xl = xs + min(rr, p.M - 1) * XS;
  const uint32_t* szl = szs + rr * GP;
  f4 acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = (f4){0.f, 0.f, 0.f, 0.f};

  for (int i0 = 0; i0 < nsw; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = i0 + d;
      if (i < nsw) {
        const int k = (i * NW + w) * KSTEP + kl;
        h2 s2[NR], z2[NR];
        if (FMT != FMT_F16) {
          const int gi = min(k >> p.gshift, p.G);  // lanes past K: zero pad entry
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const h2 v = as_h2(szl[r * RPW * GP + gi]);
            s2[r] = (h2){v.x, v.x};
            z2[r] = (h2){v.y, v.y};
          }
        }
        const _Float16* xa = xl + xswz(k);
#pragma unroll
        for (int jj = 0; jj < KPL / 8; ++jj) {
          h8 b[NR];
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const u4 v = raw[d][r];
            if (FMT == FMT_INT4) {
              const uint32_t dw = (jj == 0) ? v.x : (jj == 1) ? v.y : (jj == 2) ? v.z : v.w;
              b[r] = dq_int4_dword_perm_r(dw, s2[r], z2[r], mlo, mhi, magic);
            } else if (FMT == FMT_INT8) {
              const uint32_t d0 = (jj == 0) ? v.x : v.z;
              const uint32_t d1 = (jj == 0) ? v.y : v.w;
              h2 q0, q1, q2, q3;
              dq_int8_dword(d0, s2[r], z2[r], q0, q1);
              dq_int8_dword(d1, s2[r], z2[r], q2, q3);
              b[r].s01 = q0; b[r].s23 = q1; b[r].s45 = q2; b[r].s67 = q3;
            } else {
              b[r] = __builtin_bit_cast(h8, v);
            }
          }
          const h8 a = *(const h8*)(xa + 8 * jj);
#pragma unroll
          for (int r = 0; r < NR; ++r) acc[r] = mfma16x16x32(a, b[r], acc[r]);
        }
      }
      if (i + D < nsw) wload(i + D, d);  // uniform
    }
  }
  __syncthreads();  // all LDS activation reads done before the reduction reuses LDS

  // ---- sum the wave tiles (wave order, then shifts), epilogue ----
  // Lane holds D[m = 4*grp + e][n = nloc]; keep m / RPW == n / RPW, m % RPW < M.
  float* red = (float*)smem;                       // [NW][NR][S][M][RPW]
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * grp + e;
      if (m / RPW == sh && m % RPW < p.M)
        red[(((w * NR + r) * S + sh) * p.M + m % RPW) * RPW + rr] = acc[r][e];
    }
  __syncthreads();
  for (int idx = tid; idx < p.M * RPW; idx += NT) {
    const int im = idx / RPW, c = idx - im * RPW;
    const int row = row0 + c;
    float sum[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      sum[r] = 0.f;
      for (int ww = 0; ww < NW; ++ww)
#pragma unroll
        for (int q = 0; q < S; ++q) sum[r] += red[(((ww * NR + r) * S + q) * p.M + im) * RPW + c];
    }
    if (EPI == EPI_SWIGLU) {
      if (row < p.F) {
        const float gv = (float)(_Float16)sum[0];
        const float uv = (float)(_Float16)sum[NR - 1];
        p.C[(int64_t)im * p.ldc + row] = (_Float16)(silu_f32(gv) * uv);
      }
    } else if (row < p.N) {
      float v = sum[0];
      if (EPI == EPI_BIAS) v += (float)p.bias[row];
      p.C[(int64_t)im * p.ldc + row] = (_Float16)v;
    }
  }
}

// Chunked kernel (activations too large for LDS): chunk c holds step c*NW+w
// of every wave; the next chunk's activations are loaded into registers while
// the current chunk is consumed from LDS (two buffers, one barrier per chunk).
template <int FMT, int NW, int MB, int EPI>
__global__ __launch_bounds__(64 * NW) void gemv_chunk_kernel(GemvKArgs p) {
  constexpr int KPL = FmtTraits<FMT>::KPL;   // k per 16-byte piece
  constexpr int KSTEP = 4 * KPL;             // k per wave step
  constexpr int CHK = NW * KSTEP;            // k per chunk (one step of every wave)
  constexpr int NR = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int D = (NR == 2 || MB == 4) ? 4 : 8;
  constexpr int NT = 64 * NW;
  constexpr int CPR = CHK / 8;                           // 16-byte activation pieces per row and chunk
  constexpr int XP = (16 * MB * CPR + NT - 1) / NT;      // pieces staged per thread and chunk
  constexpr int BPK2 = (FMT == FMT_INT4) ? 1 : (FMT == FMT_INT8 ? 2 : 4);  // 2 x bytes per k
  extern __shared__ __align__(16) unsigned char smem[];
  _Float16* xs = (_Float16*)smem;
  constexpr int XS = CHK + 8;  // LDS row stride (halves), padded
  const int xbuf = p.M * XS;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nloc = lane & 15, grp = lane >> 4;
  const int r0 = 16 * blockIdx.x + nloc;
  const bool row_ok = r0 < (EPI == EPI_SWIGLU ? p.F : p.N);

  const unsigned char* wrow[NR];
  int64_t srow[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    int n = row_ok ? (r == 0 ? r0 : p.F + r0) : 0;
    wrow[r] = p.W + (int64_t)n * p.ldw;
    srow[r] = (int64_t)n * p.G;
  }

  u4 raw[D][NR];
  _Float16 sc[D][NR], zr[D][NR];
  auto wload = [&](int i, int slot) {
    const int kk = (i * NW + w) * KSTEP + grp * KPL;
    const bool ok = row_ok && kk < p.K;
    const int gi = p.gshift >= 0 ? (kk >> p.gshift) : (p.G == 1 ? 0 : kk / p.g);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      raw[slot][r] = (u4){0u, 0u, 0u, 0u};
      sc[slot][r] = (_Float16)0.f;
      zr[slot][r] = (_Float16)0.f;
      if (ok) {
        raw[slot][r] = ld16_stream(wrow[r] + (int64_t)kk * BPK2 / 2);
        if (FMT != FMT_F16) {
          sc[slot][r] = p.scales[srow[r] + gi];
          if (p.zeros) zr[slot][r] = p.zeros[srow[r] + gi];
        }
      }
    }
  };

  // activation staging (chunked mode): next chunk in registers, then LDS
  u4 xr[XP];
  auto xload = [&](int c) {
#pragma unroll
    for (int e = 0; e < XP; ++e) {
      const int idx = tid + e * NT;
      const int m = idx / CPR, cc = idx - m * CPR;
      const int kk = c * CHK + 8 * cc;
      xr[e] = (u4){0u, 0u, 0u, 0u};
      if (m < p.M && kk < p.K) xr[e] = *(const u4*)(p.A + (int64_t)m * p.lda + kk);
    }
  };
  auto xstore = [&](int buf) {
#pragma unroll
    for (int e = 0; e < XP; ++e) {
      const int idx = tid + e * NT;
      const int m = idx / CPR, cc = idx - m * CPR;
      if (m < p.M) {
        u4 v = xr[e];
        if (FMT == FMT_INT4) v = perm8_int4(v);
        *(u4*)(xs + buf * xbuf + m * XS + 8 * cc) = v;
      }
    }
  };

  // this wave's steps: i = 0 .. nsw-1 (step i is K step i*NW + w)
  const int nsw = p.nchunks;
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < nsw) wload(d, d);
  xload(0);
  xstore(0);
  __syncthreads();

  f4 acc[NR][MB];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[r][mb] = (f4){0.f, 0.f, 0.f, 0.f};

  for (int i0 = 0; i0 < nsw; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = i0 + d;
      if (i < nsw) {
        const bool more = i + 1 < nsw;
        if (more) xload(i + 1);
        // LDS row offset of this step's activations
        const _Float16* xb = xs + (i & 1) * xbuf + w * KSTEP;
        h2 s2[NR], z2[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          s2[r] = (h2){sc[d][r], sc[d][r]};
          z2[r] = (h2){zr[d][r], zr[d][r]};
        }
#pragma unroll
        for (int j = 0; j < KPL / 8; ++j) {
          h8 b[NR];
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const u4 v = raw[d][r];
            if (FMT == FMT_INT4) {
              const uint32_t dw = (j == 0) ? v.x : (j == 1) ? v.y : (j == 2) ? v.z : v.w;
              b[r] = dq_int4_dword_perm(dw, s2[r], z2[r]);
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
          const int koff = grp * KPL + 8 * j;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            const int m = 16 * mb + nloc;
            h8 a = (h8){0, 0, 0, 0, 0, 0, 0, 0};
            if (m < p.M) a = *(const h8*)(xb + m * XS + koff);
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[r][mb] = mfma16x16x32(a, b[r], acc[r][mb]);
          }
        }
        if (i + D < nsw) wload(i + D, d);
        if (more) xstore((i + 1) & 1);
        __syncthreads();
      }
    }
  }

  gemv_reduce_store<NW, NR, MB, EPI>(p, acc, smem, tid, w, nloc, grp);
}

template <typename KFn>
hipError_t launch_kernel(KFn fn, const GemvKArgs& k, int rowblocks, int threads, size_t lds, hipStream_t s,
                         bool& attr_set) {
  if (!attr_set && lds > 65536) {  // raise the dynamic LDS limit once per instantiation
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(fn, dim3(rowblocks), dim3(threads), lds, s, k);
  return hipGetLastError();
}

template <int FMT, int NW, int RPW, int EPI>
hipError_t launch_full(const GemvKArgs& k, const GemvPlan& p, hipStream_t s) {
  constexpr int D = (EPI == EPI_SWIGLU) ? 8 : 16;  // weight ring depth
  static bool attr = false;
  return launch_kernel(gemv_full_kernel<FMT, NW, RPW, EPI, D>, k, p.rowblocks, 64 * NW, p.lds_bytes, s, attr);
}

template <int FMT, int NW, int MB, int EPI>
hipError_t launch_chunk(const GemvKArgs& k, const GemvPlan& p, hipStream_t s) {
  static bool attr = false;
  return launch_kernel(gemv_chunk_kernel<FMT, NW, MB, EPI>, k, p.rowblocks, 64 * NW, p.lds_bytes, s, attr);
}

template <int FMT, int EPI>
hipError_t dispatch_full(const GemvKArgs& k, const GemvPlan& p, hipStream_t s) {
#define MQ_FULL(NW_, RPW_) \
  if (p.nw == NW_ && p.rpw == RPW_) return launch_full<FMT, NW_, RPW_, EPI>(k, p, s);
  MQ_FULL(4, 2) MQ_FULL(4, 4) MQ_FULL(4, 8) MQ_FULL(4, 16)
  MQ_FULL(8, 2) MQ_FULL(8, 4) MQ_FULL(8, 8) MQ_FULL(8, 16)
  MQ_FULL(16, 2) MQ_FULL(16, 4) MQ_FULL(16, 8) MQ_FULL(16, 16)
#undef MQ_FULL
  return hipErrorInvalidValue;
}

template <int FMT, int EPI>
hipError_t dispatch_chunk(const GemvKArgs& k, const GemvPlan& p, hipStream_t s) {
#define MQ_CHUNK(NW_, MB_) \
  if (p.nw == NW_ && p.mblocks == MB_) return launch_chunk<FMT, NW_, MB_, EPI>(k, p, s);
  MQ_CHUNK(2, 1) MQ_CHUNK(2, 2) MQ_CHUNK(2, 4)
  MQ_CHUNK(4, 1) MQ_CHUNK(4, 2) MQ_CHUNK(4, 4)
  MQ_CHUNK(8, 1) MQ_CHUNK(8, 2) MQ_CHUNK(8, 4)
  MQ_CHUNK(16, 1) MQ_CHUNK(16, 2) MQ_CHUNK(16, 4)
#undef MQ_CHUNK
  return hipErrorInvalidValue;
}

template <int FMT>
hipError_t dispatch(const GemvKArgs& k, const GemvPlan& p, int epi, hipStream_t s) {
  if (FMT == FMT_F16 || epi == EPI_NONE)
    return p.xfull ? dispatch_full<FMT, EPI_NONE>(k, p, s) : dispatch_chunk<FMT, EPI_NONE>(k, p, s);
  if (epi == EPI_BIAS)
    return p.xfull ? dispatch_full<FMT, EPI_BIAS>(k, p, s) : dispatch_chunk<FMT, EPI_BIAS>(k, p, s);
  return p.xfull ? dispatch_full<FMT, EPI_SWIGLU>(k, p, s) : dispatch_chunk<FMT, EPI_SWIGLU>(k, p, s);
}

int kpl_of(int fmt) { return fmt == FMT_INT4 ? 32 : (fmt == FMT_INT8 ? 16 : 8); }

}  // namespace

bool gemv_supported(const LinearArgs& a) {
  const int kpl = kpl_of(a.fmt);
  if (a.M < 1 || a.M > 64) return false;
  if (a.K % kpl != 0) return false;                        // whole 16-byte pieces per row
  if (a.fmt != FMT_F16 && (a.g % kpl != 0)) return false;  // one group per piece
  if (a.fmt != FMT_F16 && (a.g & (a.g - 1)) && a.G != 1) return false;  // group index by shift
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  return true;
}

GemvPlan gemv_plan(const LinearArgs& a, const GemvTuning& t) {
  GemvPlan p{};
  const int kpl = kpl_of(a.fmt);
  const int nr = a.epi == EPI_SWIGLU ? 2 : 1;
  const int nrows = a.epi == EPI_SWIGLU ? a.F : a.N;
  // whole-K kernel: M <= RPW <= 16 and the activations fit in LDS
  if (t.allow_full && a.M <= 16 && a.G < 65536) {
    int rpw = t.rpw ? t.rpw : (a.M <= 4 ? 4 : (a.M <= 8 ? 8 : 16));
    if (rpw < a.M) rpw = 16;
    const int s = 16 / rpw;
    const int kstep = 4 * kpl * s;
    const int nsteps = (a.K + kstep - 1) / kstep;
    const int kpad = nsteps * kstep;
    const int xs_stride = ((kpad + 127) / 128) * 136 + 8;
    int nw = 16;  // widest workgroup that still gives every wave several steps
    while (nw > 4 && (nw > t.max_nw || nsteps < 4 * nw)) nw >>= 1;
    const size_t xbytes = (size_t)a.M * xs_stride * 2 + (size_t)nr * rpw * (a.G + 1) * 4;
    const size_t rbytes = (size_t)nw * nr * s * a.M * rpw * 4;
    const size_t lds = xbytes > rbytes ? xbytes : rbytes;
    if (lds <= 163840) {
      p.xfull = true;
      p.rpw = rpw;
      p.nw = nw;
      p.mblocks = 1;
      p.nsteps = nsteps;
      p.kpad = kpad;
      p.nchunks = 0;
      p.rowblocks = (nrows + rpw - 1) / rpw;
      p.xs_stride = xs_stride;
      p.lds_bytes = lds;
      return p;
    }
  }
  // chunked kernel: two chunk buffers of activations in LDS
  const int kstep = 4 * kpl;
  const int nsteps = (a.K + kstep - 1) / kstep;
  p.xfull = false;
  p.rpw = 16;
  p.mblocks = a.M <= 16 ? 1 : (a.M <= 32 ? 2 : 4);
  p.rowblocks = (nrows + 15) / 16;
  int nw = 16;
  while (nw > 2) {
    size_t lds = 2ull * a.M * (nw * kstep + 8) * 2;
    if (nw <= t.max_nw && lds <= 131072 && nw <= nsteps) break;
    nw >>= 1;
  }
  p.nw = nw;
  p.nsteps = nsteps;
  p.kpad = nsteps * kstep;
  p.nchunks = (nsteps + nw - 1) / nw;
  size_t xbytes = 2ull * a.M * (nw * kstep + 8) * 2;
  size_t rbytes = (size_t)nw * nr * a.M * 16 * 4;
  p.lds_bytes = xbytes > rbytes ? xbytes : rbytes;
  return p;
}

hipError_t gemv_launch(const LinearArgs& a, const GemvPlan& p, hipStream_t s) {
  GemvKArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.bias = (const _Float16*)a.bias;
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.g = a.g > 0 ? a.g : 1; k.G = a.G; k.F = a.F;
  k.gshift = -1;
  for (int b = 0; b < 31; ++b)
    if (k.g == (1 << b)) k.gshift = b;
  k.nchunks = p.nchunks;
  k.nsteps = p.nsteps;
  k.kpad = p.kpad;
  k.xs_stride = p.xs_stride;
  {  // floor(x / d) = (x * ceil(2^40 / d)) >> 40 exactly for x < 2^24, d <= 2^16
    const uint64_t dvs = (uint64_t)(a.G + 1);
    k.gp_m64 = ((1ull << 40) + dvs - 1) / dvs;
  }
  k.mlo = 0x000F000Fu;
  k.mhi = 0x00F000F0u;
  k.magic = 0x64006400u;
  if (k.gshift < 0) k.gshift = (k.G == 1) ? 31 : -1;  // one group spanning K: index is always 0
  switch (a.fmt) {
    case FMT_INT4: return dispatch<FMT_INT4>(k, p, a.epi, s);
    case FMT_INT8: return dispatch<FMT_INT8>(k, p, a.epi, s);
    default: return dispatch<FMT_F16>(k, p, a.epi, s);
  }
}

}  // namespace mq
