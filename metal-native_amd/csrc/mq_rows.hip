// Persistent row-block MFMA GEMV for skinny activations whose activation rows
// fit in LDS (decode; the Qwen2.5-7B down-proj at M = 1 is its main case).
//
// Replaces, like mq_gemv.hip, the reference's M<=8 routes
// (shaders/matmul_dequant_kernel.metal:229-345, :485-576, dispatched at
// src/ops/matmul.mm:946-1009; shaders/matmul_vecmat_kernel.metal:32-139 for
// fp16 B [N, K]), computing every row of A.
//
// Structure (one launch; no workgroup waits for another):
//  * One workgroup of NW (12, or 8 for small problems) wavefronts per CU.  Workgroup b owns R consecutive
//    output rows (SwiGLU: R output columns = R gate + R up weight rows) over
//    the whole of K, so every CU streams the same number of weight bytes.
//    When the activations of all of K do not fit in LDS (M = 4 at K = 18944),
//    K is cut into KP contiguous parts: one workgroup per (row block, part),
//    with KP times the rows, and the parts of a row block meet through the
//    workspace (the last to arrive sums them in K order).
//  * Row tile: RPW weight rows x S = 16/RPW K shifts form the 16 columns of the
//    B operand of v_mfma_f32_16x16x32_f16; one wave load reads RPW rows x 64*S
//    contiguous bytes.  The A operand holds activation row i % RPW at K shift
//    i / RPW (needs M <= RPW; RPW = 8 and 16 only for the quantized formats); the
//    result for (activation i, weight row r) is sum_s D[s*RPW + i][s*RPW + r].
//    M = 9..16 (quantized, no pre-norm) runs on 8-row tiles with the
//    activation rows in two halves: each dequantized fragment feeds two
//    MFMAs, rows 0..7 and 8..15 (16-row tiles would read only 64 bytes of each
//    of 16 rows per load, and cost 13 % more at config 4, M = 16).
//  * The workgroup's work is TW tiles x KS K-steps ("units", tile-major); wave
//    w takes the contiguous units [w*U/NW, (w+1)*U/NW) and streams them
//    through a ring of D register slots refilled as they are consumed.  Every
//    load is an unconditional buffer load (units past the wave's range use an
//    out-of-range offset), so the load counter is exact and each unit waits
//    for its own slot only; compute overlaps the stream.
//  * The activations (all of K, re-ordered for the int4 operand layout) and
//    the scales/zeros of the workgroup's rows are staged in LDS once.  Their
//    loads go out first and are waited for after only a short head of the
//    weight stream: a wave stalls at issue while the memory queues are full,
//    so a deep stream issued first would hold back the start of compute.
//  * When a tile ends (or the wave's range does) the wave folds the K shifts
//    of its accumulator through a per-wave LDS scratch and stores the tile's
//    M x RPW partial in its own slot.  At the end the workgroup sums, for
//    each output, the slots of the waves that touched its tile in wave order
//    (deterministic), applies the epilogue and stores fp16.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <algorithm>
#include <cmath>

namespace mq {
namespace {

// ring depth (units in flight per wave): 3 for int4, whose loop is bound by
// the dequant issue (config 2 M=1: 11.6-11.8 vs 11.9-12.4 us with 4, M=4
// 15.1-15.3 vs 15.5-15.7), 4 for int8 and fp16, which wait on the stream
// (config 4 M=1: 25.8-26.3 vs 26.1-26.6 us with 3; 2 is slower for both)
template <int FMT>
constexpr int ring_depth() { return FMT == FMT_INT4 ? 3 : 4; }
// wavefronts per workgroup: 12, or 8 when the workgroup streams at most
// kSmallBytes of weights (measured at M = 1: 8 waves 4-8 % faster at 2-8 MB
// in total, 3-4 % slower at 34 MB and more)
constexpr int kNWBig = 12, kNWSmall = 8;
constexpr int64_t kSmallBytes = 64 * 1024;
static_assert(kNWBig % 4 == 0 && kNWSmall % 4 == 0, "the slot sums read the first-tile table in groups of four");
constexpr int kPre = 2;      // ring slots issued before the staging data is waited for
constexpr int kXB = 8;           // activation pieces per thread per staging batch
constexpr int kSB = 2;           // scale/zero pieces per thread per staging batch
constexpr size_t kLds = 163840;  // LDS per CU on gfx950
constexpr size_t kCntBytesRows = 65536;   // workspace counters (the split-K GEMV's layout)

struct RowsKArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros;
  EpiArgs ep;     // element-wise epilogue (kernels without SwiGLU)
  _Float16* C; int64_t ldc;
  int M, K, N, F, G, gshift;
  int R;          // output rows (SwiGLU: output columns) per workgroup
  int TW;         // row tiles per workgroup
  int KS;         // K steps per part (staged width; the last part may have fewer)
  int KStot;      // K steps per row
  int KP, nblk;   // K parts, row blocks (grid = KP * nblk)
  float* part;    // KP > 1: fp32 partial outputs [KP][nblk][M * R * (SwiGLU ? 2 : 1)]
  uint32_t* cnt;  // KP > 1: arrivals per row block (zero between launches)
  int XS;         // LDS activation row stride (halves)
  int maxT;       // partial slots per wave
  int snp;        // 16-byte scale pieces staged per region (one, or two for SwiGLU)
  uint32_t off_sz, off_scr, off_slot, off_wft;  // LDS byte offsets
  uint32_t sz_bytes, z_bytes;
  const _Float16* pre_delta; const _Float16* pre_weight; _Float16* pre_resid;  // fused pre-norm (PRE)
  float pre_eps;
};

template <int FMT, int EPI, int RPW, bool PRE, int NW, int MH>
__global__ __launch_bounds__(64 * NW) void rows_kernel(RowsKArgs p) {
  constexpr int S = 16 / RPW;
  constexpr int KPL = FmtTraits<FMT>::KPL;       // k per 16-byte piece
  constexpr int KSTEP = 4 * KPL * S;             // k per row per unit
  constexpr int NJ = KPL / 8;                    // MFMAs per unit
  constexpr int HALF = RPW / 2;
  constexpr int BPK2 = (FMT == FMT_INT4) ? 1 : (FMT == FMT_INT8 ? 2 : 4);  // 2 x bytes per k
  extern __shared__ __align__(16) unsigned char smem[];

  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // K part kpi of row block b: steps [ks0, ks0 + KS) of the row
  const int kpi = blockIdx.x / p.nblk, b = blockIdx.x - kpi * p.nblk;
  const int ks0 = kpi * p.KS;
  const int M = p.M, KS = min(p.KStot - ks0, p.KS);

  _Float16* xs = (_Float16*)smem;                     // [M][XS]
  uint32_t* szl = (uint32_t*)(smem + p.off_sz);       // [regions][8 snp]: s | z << 16
  float* scr = (float*)(smem + p.off_scr) + w * 256;  // per wave [16][16]
  float* slots = (float*)(smem + p.off_slot);         // [NW][maxT][M*RPW]
  int* wft = (int*)(smem + p.off_wft);                // [NW] first tile of each wave's unit range

  const int nl = lane & 15, gi = lane >> 4;
  const int r = nl % RPW, sh = nl / RPW;              // weight row in tile, K shift
  const int klane = sh * 4 * KPL + gi * KPL;          // this lane's k within a unit

  // ---- this workgroup's weight rows ----
  // local weight row lr: plain lr = t*RPW + r (global row0 + lr); SwiGLU the
  // tile holds gate columns c = t*HALF + r (r < HALF) and the matching up
  // rows, local rows c and R + c (global f0 + c and F + f0 + c).
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
  const rsrc_t wr = make_rsrc(p.W + (int64_t)row0 * p.ldw, span);
  auto row_off = [&](int t) -> uint32_t {  // byte offset of this lane's row of tile t, or kOob
    if (EPI == EPI_SWIGLU) {
      const int c = t * HALF + (r % HALF);
      if (c >= valid) return kOob;
      return (uint32_t)(((r < HALF) ? c : p.F + c) * p.ldw);
    } else {
      const int lr = t * RPW + r;
      return lr < valid ? (uint32_t)(lr * p.ldw) : kOob;
    }
  };

  // ---- unit range of this wave and the ring ----
  const int U = p.TW * KS;
  const int u0 = (w * U) / NW;   // NW is a compile-time constant: no division instruction
  const int nu = ((w + 1) * U) / NW - u0;
  int lt = u0 / KS, lj = u0 - lt * KS;   // load cursor (tile, step)
  int left = nu;                          // units the load cursor has not issued
  // Load offset = lane part (row of tile lt + the lane's k) + step part
  // (uniform: the buffer instruction's scalar offset).  Only the last step
  // checks k against K per lane.  Out-of-range parts use kOobPart, so a sum
  // of two still fails the range check.
  constexpr uint32_t kOobPart = 0x40000000u;
  auto lane_off = [&](int t) -> uint32_t {
    const uint32_t ro = row_off(t);
    return ro == kOob ? kOobPart : ro + (uint32_t)(klane * BPK2 / 2);
  };
  // fp16 weights: the last step reads no bytes past K (raw fp16 there may
  // hold any bits); its lane part is lvo_last.  Quantized bytes past K (the
  // next row's, row padding, or zeros past the range) dequantize to finite
  // values that meet zero activations, so those lanes load unmasked.
  const bool kpast = FMT == FMT_F16 && (ks0 + KS - 1) * KSTEP + klane >= p.K;
  uint32_t lvo = lane_off(lt), lvo_last = kpast ? kOobPart : lvo;
  auto wload = [&]() -> u4 {
    uint32_t so = kOobPart, vo = lvo;
    if (left > 0) {
      so = (uint32_t)((ks0 + lj) * (KSTEP * BPK2 / 2));
      if (FMT == FMT_F16 && lj == KS - 1) vo = lvo_last;
      --left;
      if (++lj == KS) {
        lj = 0;
        ++lt;
        lvo = lane_off(lt);
        if (FMT == FMT_F16) lvo_last = kpast ? kOobPart : lvo;
      }
    }
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wr, vo, so, 2));
  };

  // ---- staging loads, issued before the ring: the load counter completes
  // in order, so staging data loaded after the ring would wait for it.
  // Every per-thread offset is a lane part computed once plus a uniform
  // part: the staging runs on 3 waves per SIMD before the stream starts, so
  // its VALU work is paid in full at the start of every launch ----
  // activations: thread tid stages pieces c = tid + j*NT (j < epr) of each
  // row i; one buffer resource per row, K*2 bytes long, so pieces past K
  // read zeros
  const int ppr = p.KS * KSTEP / 8;    // pieces per staged row (the widest part)
  const int kx0 = ks0 * KSTEP / 8;     // the part's first 16-byte piece of a row
  const int epr = (ppr + NT - 1) / NT;  // loads per row per thread
  const int nxs = M * epr;              // staging slots per thread
  const int nxb = min(kXB, nxs);
  const uint32_t xvo = (uint32_t)(kx0 + tid) * 16u;                  // global offset, lane part
  const uint32_t xlo = (uint32_t)(16 * tid + 16 * (tid >> 4));       // LDS offset of xswz(8 tid), bytes
  auto x_row = [&](int i) { return make_rsrc(p.A + (int64_t)i * p.lda, (uint32_t)(p.K * 2)); };
  auto x_fetch = [&](int s0, u4* v, int cnt) {
    int i = s0 / epr, j = s0 - i * epr;   // uniform
#pragma unroll
    for (int e = 0; e < kXB; ++e) {
      if (e < cnt) {
        v[e] = bload16(x_row(min(i, M - 1)), s0 + e < nxs ? xvo + (uint32_t)(j * NT * 16) : kOob);
        if (++j == epr) { j = 0; ++i; }
      }
    }
  };
  auto x_put = [&](int s0, const u4* v, int cnt) {
    int i = s0 / epr, j = s0 - i * epr;
#pragma unroll
    for (int e = 0; e < kXB; ++e) {
      if (e < cnt && s0 + e < nxs) {
        if (tid + j * NT < ppr) {
          u4 vv = v[e];
          if (FMT == FMT_INT4) vv = perm8_int4(vv);
          *(u4*)((unsigned char*)xs + i * p.XS * 2 + xlo + j * NT * 17) = vv;
        }
        if (++j == epr) { j = 0; ++i; }
      }
    }
  };
  // scales/zeros, as s | z << 16 dwords: region 0 holds the 16-byte pieces
  // of the [N][G] arrays that cover the entries of rows row0 .. row0+R-1
  // plus the kstep/g entries that steps past K read (region 1, SwiGLU: the
  // up rows F+row0 ..), copied whole from the piece boundary below the
  // rows' first entry.  Entries outside the rows (the neighbouring rows',
  // or zeros past the arrays) feed only rows past N, whose outputs are not
  // stored: lanes past K keep their own row's last entry (below).
  const rsrc_t sr = make_rsrc(p.scales, p.sz_bytes);
  const rsrc_t zr = make_rsrc(p.zeros, p.z_bytes);
  const int G = p.G;
  const uint32_t sz_real = (uint32_t)p.N * (uint32_t)G * 2u;  // bytes of the scale array
  const int snp = p.snp;                                      // pieces per region
  const int eb0 = row0 * G;                                   // first entry of region 0
  const int eb1 = (EPI == EPI_SWIGLU ? p.F + row0 : 0) * G;   // first entry of region 1
  const int pb0 = eb0 >> 3, pb1 = eb1 >> 3;
  const int sb0 = eb0 & 7, sb1 = 8 * snp + (eb1 & 7);         // LDS entry of each region's first row
  const int nps = FMT != FMT_F16 ? (EPI == EPI_SWIGLU ? 2 : 1) * snp : 0;
  const int nsb = min(kSB, (nps + NT - 1) / NT);
  auto s_fetch = [&](int base, u4* sv, u4* zv, int cnt) {
#pragma unroll
    for (int e = 0; e < kSB; ++e) {
      if (e < cnt) {
        const int idx = base + tid + e * NT;
        const int gp = idx < snp ? pb0 + idx : pb1 - snp + idx;
        const uint32_t off = idx < nps ? (uint32_t)gp * 16u : kOob;
        if (off == kOob || off + 16u <= sz_real) {
          sv[e] = bload16(sr, off);
          zv[e] = bload16(zr, off);
        } else {  // the piece that straddles the end of the arrays: entry by entry
          uint32_t sw[4], zw[4];
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const uint32_t o0 = off + 4u * h, o1 = o0 + 2u;
            const uint32_t q0 = o0 < sz_real ? o0 : kOob, q1 = o1 < sz_real ? o1 : kOob;
            sw[h] = bload2(sr, q0) | (bload2(sr, q1) << 16);
            zw[h] = bload2(zr, q0) | (bload2(zr, q1) << 16);
          }
          sv[e] = (u4){sw[0], sw[1], sw[2], sw[3]};
          zv[e] = (u4){zw[0], zw[1], zw[2], zw[3]};
        }
      }
    }
  };
  auto s_put = [&](int base, const u4* sv, const u4* zv, int cnt) {
#pragma unroll
    for (int e = 0; e < kSB; ++e) {
      const int idx = base + tid + e * NT;
      if (e < cnt && idx < nps) {
        const u4 a = sv[e], z = zv[e];
        *(u4*)(szl + 8 * idx) = (u4){__builtin_amdgcn_perm(z.x, a.x, 0x05040100u), __builtin_amdgcn_perm(z.x, a.x, 0x07060302u),
                                     __builtin_amdgcn_perm(z.y, a.y, 0x05040100u), __builtin_amdgcn_perm(z.y, a.y, 0x07060302u)};
        *(u4*)(szl + 8 * idx + 4) = (u4){__builtin_amdgcn_perm(z.z, a.z, 0x05040100u), __builtin_amdgcn_perm(z.z, a.z, 0x07060302u),
                                         __builtin_amdgcn_perm(z.w, a.w, 0x05040100u), __builtin_amdgcn_perm(z.w, a.w, 0x07060302u)};
      }
    }
  };

  constexpr int kD = ring_depth<FMT>();
  u4 raw[kD];
  {
    u4 xv[kXB];
    u4 sv[kSB], zv[kSB];
    u4 dv[PRE ? kXB : 1], wv[PRE ? kXB : 1];
    x_fetch(0, xv, nxb);
    if (PRE) {  // residual delta and norm weight pieces, same indices (M = 1: piece c at 16c bytes)
      const rsrc_t dr = make_rsrc(p.pre_delta, p.pre_delta ? (uint32_t)(p.K * 2) : 0u);
      const rsrc_t nr = make_rsrc(p.pre_weight, (uint32_t)(p.K * 2));
#pragma unroll
      for (int e = 0; e < kXB; ++e) {
        if (e < nxb) {
          const uint32_t off = xvo + (uint32_t)(e * NT * 16);   // M = 1, one part: slot e is piece tid + e*NT
          dv[e] = bload16(dr, off);
          wv[e] = bload16(nr, off);
        }
      }
    }
    if (FMT != FMT_F16) s_fetch(0, sv, zv, nsb);
    // Then a short head of the weight stream.  The staging data is waited
    // for before the rest: a wave blocks while the memory queues are full, so
    // a deep stream issued first would hold back the start of compute.
#pragma unroll
    for (int d = 0; d < kPre; ++d) raw[d] = wload();
#pragma unroll
    for (int e = 0; e < kXB; ++e) asm volatile("" : "+v"(xv[e]));
#pragma unroll
    for (int e = 0; e < kSB; ++e) asm volatile("" : "+v"(sv[e]), "+v"(zv[e]));
    if (PRE) {
      // A' = half(A + delta) (the residual, stored by workgroup 0), then the
      // row's sum of squares across the workgroup, then the normalised pieces
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < kXB; ++e) {
        if (e < nxb) {
          asm volatile("" : "+v"(dv[e]), "+v"(wv[e]));
          h8 v = __builtin_bit_cast(h8, xv[e]);
          if (p.pre_delta) {
            const h8 d = __builtin_bit_cast(h8, dv[e]);
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = (_Float16)((float)v[k] + (float)d[k]);
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) ss += (float)v[k] * (float)v[k];
          xv[e] = __builtin_bit_cast(u4, v);
          const int idx = tid + e * NT;
          if (b == 0 && idx < ppr && 8 * idx < p.K) *(h8*)(p.pre_resid + 8 * idx) = v;
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ss += xor_lane(ss, o);
      float* red = (float*)(smem + p.off_scr);   // per-wave scratch, free until the first tile fold
      if (lane == 0) red[w * 256] = ss;
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      float tot = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) tot += red[ww * 256];
      const float rn = rsqrtf(tot / (float)p.K + p.pre_eps);
#pragma unroll
      for (int e = 0; e < kXB; ++e) {
        if (e < nxb) {
          const h8 v = __builtin_bit_cast(h8, xv[e]);
          const h8 wn = __builtin_bit_cast(h8, wv[e]);
          h8 o8;
#pragma unroll
          for (int k = 0; k < 8; ++k) o8[k] = (_Float16)((float)v[k] * rn * (float)wn[k]);
          xv[e] = __builtin_bit_cast(u4, o8);
        }
      }
    }
    x_put(0, xv, nxb);
    if (FMT != FMT_F16) s_put(0, sv, zv, nsb);
  }
  // the rest (large M*K, many scale rows), then the rest of the ring: loads
  // complete in order, so staging loads issued behind the ring would wait
  // for its weights
  for (int s0 = kXB; s0 < nxs; s0 += kXB) {
    u4 xv[kXB];
    x_fetch(s0, xv, kXB);
    x_put(s0, xv, kXB);
  }
  for (int base = kSB * NT; base < nps; base += kSB * NT) {
    u4 sv[kSB], zv[kSB];
    s_fetch(base, sv, zv, kSB);
    s_put(base, sv, zv, kSB);
  }
#pragma unroll
  for (int d = kPre; d < kD; ++d) raw[d] = wload();
  // LDS barrier that leaves the weight loads in flight
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // ---- stream ----
  // MH activation-row halves (MH = 2: M = 9..16 on 8-row tiles, the second
  // half's fragments RPW rows further down, the same dequantized weights)
  const int xrow = min(r, M - 1) * p.XS;
  const int xdh = (min(r + RPW, M - 1) - min(r, M - 1)) * p.XS;
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u;
  asm volatile("" : "+v"(mlo), "+v"(mhi));  // keep the nibble masks in VGPRs
  const uint32_t magic = 0x64006400u;

  int ct = u0 / KS, cj = u0 - ct * KS;   // consume cursor (tile, step)
  const int ft = ct;                      // first tile of this wave
  if (lane == 0) wft[w] = ft;   // read by the slot sums after the final barrier
  // scale entry of the lane's row and group: the step advances it by a
  // uniform KSTEP / g groups.  In a row's last step, lanes whose k lies past
  // K would reach the next row's entries: they keep their own row's last
  // entry instead (the weights there meet zero activations, and a row's
  // output must not depend on another row's scales, finite or not).
  const int sadv = p.gshift >= 31 ? 0 : (KSTEP >> p.gshift);
  const int sl = p.gshift >= 31 ? 0 : (klane >> p.gshift);
  // LDS entry of this lane's row of tile t, group 0
  auto sz_ent = [&](int t) -> int {
    if (EPI == EPI_SWIGLU) {
      const int c = t * HALF + (r % HALF);
      return ((r < HALF) ? sb0 : sb1) + c * G;
    }
    return sb0 + (t * RPW + r) * G;
  };
  int sa = sz_ent(ct) + sl + (ks0 + cj) * sadv;
  auto clamp_last = [&]() {   // uniform condition: the row's last step
    if (FMT != FMT_F16 && ks0 + cj == p.KStot - 1) sa = min(sa, sz_ent(ct) + G - 1);
  };
  clamp_last();
  const _Float16* xa = xs + xrow + xswz(cj * KSTEP + klane);
  // the LDS activation padding (8 halves per 128) advances by a constant per
  // unit when a unit spans whole 128-k blocks; otherwise (16-row int8 tiles,
  // 64 k per unit) the fragment address is recomputed per unit
  constexpr bool XCONST = KSTEP % 128 == 0;
  constexpr int XADV = KSTEP + (KSTEP >> 7) * 8;
  f4 acc[MH];
#pragma unroll
  for (int h = 0; h < MH; ++h) acc[h] = (f4){0.f, 0.f, 0.f, 0.f};

  auto flush = [&]() {
#pragma unroll
    for (int h = 0; h < MH; ++h) {
      mfma_result_fence(acc[h]);
#pragma unroll
      for (int e = 0; e < 4; ++e) scr[(4 * gi + e) * 16 + nl] = acc[h][e];
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const int mh = min(M - RPW * h, RPW);   // activation rows of this half
      for (int idx = lane; idx < mh * RPW; idx += 64) {   // one pass but for 16-row tiles
        const int i = idx / RPW, rr = idx - i * RPW;
        float v = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) v += scr[(s * RPW + i) * 16 + s * RPW + rr];
        slots[(w * p.maxT + (ct - ft)) * (M * RPW) + RPW * RPW * h + idx] = v;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      acc[h] = (f4){0.f, 0.f, 0.f, 0.f};
    }
  };

  auto step = [&](const u4 v) {
    h2 s2 = (h2){(_Float16)0.f, (_Float16)0.f}, z2 = s2;
    if (FMT != FMT_F16) {
      // broadcast halves: the packed ops' operand selectors read them in place
      const h2 e = as_h2(szl[sa]);
      s2 = __builtin_shufflevector(e, e, 0, 0);
      z2 = __builtin_shufflevector(e, e, 1, 1);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      h8 bq;
      if (FMT == FMT_INT4) {
        const uint32_t dw = (j == 0) ? v.x : (j == 1) ? v.y : (j == 2) ? v.z : v.w;
        bq = dq_int4_dword_perm_r(dw, s2, z2, mlo, mhi, magic);
      } else if (FMT == FMT_INT8) {
        const uint32_t d0 = (j == 0) ? v.x : v.z;
        const uint32_t d1 = (j == 0) ? v.y : v.w;
        h2 q0, q1, q2, q3;
        dq_int8_dword(d0, s2, z2, q0, q1);
        dq_int8_dword(d1, s2, z2, q2, q3);
        bq.s01 = q0; bq.s23 = q1; bq.s45 = q2; bq.s67 = q3;
      } else {
        bq = __builtin_bit_cast(h8, v);
      }
#pragma unroll
      for (int h = 0; h < MH; ++h) {
        const h8 a = *(const h8*)(xa + h * xdh + 8 * j);
        acc[h] = mfma16x16x32(a, bq, acc[h]);
      }
    }
  };

  // wave priority falls with progress (the arbiter issues from the highest
  // priority ready wave): the waves of a SIMD advance together, so the last
  // units are not left to one wave that cannot hide the load latency alone
  __builtin_amdgcn_s_setprio(3);
  const int q1 = nu >> 2, q2 = nu >> 1, q3 = (3 * nu) >> 2;
  for (int base = 0; base < nu; base += kD) {
#pragma unroll
    for (int d = 0; d < kD; ++d) {
      if (base + d < nu) {
        if (base + d == q1) __builtin_amdgcn_s_setprio(2);
        if (base + d == q2) __builtin_amdgcn_s_setprio(1);
        if (base + d == q3) __builtin_amdgcn_s_setprio(0);
        step(raw[d]);
        if constexpr (XCONST) xa += XADV;
        sa += sadv;
        const bool last = base + d == nu - 1;
        if (++cj == KS || last) {
          flush();
          if (cj == KS) {
            cj = 0;
            ++ct;
            xa = xs + xrow + xswz(klane);
            sa = sz_ent(ct) + sl + ks0 * sadv;
          }
        }
        if constexpr (!XCONST) xa = xs + xrow + xswz(cj * KSTEP + klane);
        clamp_last();
      }
      raw[d] = wload();
    }
  }
  __syncthreads();

  // ---- sum the slots per output, epilogue ----
  const int MR = M * RPW;
  auto tile_sum = [&](int t, int i, int rr) -> float {
    // Every wave's first tile and slot entry are read unconditionally (the
    // index of a wave that did not touch the tile is masked to entry 0, its
    // value to +0), so the reads are in flight together instead of one LDS
    // round trip per wave; the sum keeps wave order, and adding +0 to a sum
    // that starts at +0 leaves it bit-identical.
    const int ub = t * KS, ue = ub + KS;
    int fw[NW];
#pragma unroll
    for (int ww = 0; ww < NW; ww += 4) {
      const int4 f4 = *(const int4*)(wft + ww);
      fw[ww] = f4.x; fw[ww + 1] = f4.y; fw[ww + 2] = f4.z; fw[ww + 3] = f4.w;
    }
    float sv[NW];
    bool use[NW];
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const int a0 = (ww * U) / NW, a1 = ((ww + 1) * U) / NW;
      use[ww] = a0 < ue && a1 > ub && a1 > a0;
      const int idx = ((ww * p.maxT + (t - fw[ww])) * MR + i * RPW + rr) & -(int)use[ww];
      sv[ww] = slots[idx];
    }
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) v += use[ww] ? sv[ww] : 0.f;
    return v;
  };
  if (p.KP > 1) {
    // ---- K parts: partial outputs through the workspace; the last part of
    // the row block to arrive sums them in K order ----
    // Ordering: every access to the partials is a system-scope atomic
    // (stores written through to memory, loads served from memory) and a
    // workgroup's stores are acknowledged (s_waitcnt vmcnt(0)) before its
    // arrival is counted: the release/acquire of the split-K GEMV's
    // protocol.  No workgroup waits for another.
    constexpr int PV = EPI == EPI_SWIGLU ? 2 : 1;
    const int64_t pstride = (int64_t)p.nblk * M * p.R * PV;   // one part
    float* const pown = p.part + (int64_t)kpi * pstride + (int64_t)b * M * p.R * PV;
    auto own = [&](int idx, int e) -> float {   // this part's sum: output idx, gate (0) or up (1)
      const int i = idx / valid, c = idx - i * valid;
      if (EPI == EPI_SWIGLU) {
        const int t = c / HALF, rr = c - t * HALF;
        return tile_sum(t, i, rr + e * HALF);
      }
      const int t = c / RPW, rr = c - t * RPW;
      return tile_sum(t, i, rr);
    };
    for (int idx = tid; idx < M * valid; idx += NT)
#pragma unroll
      for (int e = 0; e < PV; ++e)
        __hip_atomic_store(pown + idx * PV + e, own(idx, e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // the arrival flag lives in the per-wave scratch (free since the last
    // fold; a static __shared__ variable would shrink the dynamic LDS the
    // kernel may request)
    volatile uint32_t* s_last = (volatile uint32_t*)(smem + p.off_scr);
    if (tid == 0)
      *s_last = __hip_atomic_fetch_add(p.cnt + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == (uint32_t)(p.KP - 1);
    __syncthreads();
    if (!*s_last) return;
    for (int idx = tid; idx < M * valid; idx += NT) {
      float v[PV];
#pragma unroll
      for (int e = 0; e < PV; ++e) {
        v[e] = 0.f;
        for (int kp = 0; kp < p.KP; ++kp)   // K order, whatever the arrival order
          v[e] += kp == kpi ? own(idx, e) : ld_coherent(pown + (int64_t)(kp - kpi) * pstride + idx * PV + e);
      }
      const int i = idx / valid, c = idx - i * valid;
      if (EPI == EPI_SWIGLU)
        p.C[(int64_t)i * p.ldc + row0 + c] = (_Float16)(silu_f32((float)(_Float16)v[0]) * (float)(_Float16)v[PV - 1]);
      else
        p.C[(int64_t)i * p.ldc + row0 + c] = (_Float16)epi_apply(v[0], i, row0 + c, p.ep);
    }
    if (tid == 0) __hip_atomic_store(p.cnt + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return;
  }
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

template <int FMT, int EPI, int RPW, bool PRE, int NW, int MH>
hipError_t launch5(const RowsKArgs& k, const RowsPlan& pl, hipStream_t s) {
  auto fn = rows_kernel<FMT, EPI, RPW, PRE, NW, MH>;
  hipError_t e = allow_dynamic_lds((const void*)fn, (int)kLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(fn, dim3(pl.nwg), dim3(64 * NW), pl.lds_bytes, s, k);
  return hipGetLastError();
}

template <int FMT, int EPI, int RPW, bool PRE>
hipError_t launch4(const RowsKArgs& k, const RowsPlan& pl, hipStream_t s) {
  if constexpr (RPW == 8 && !PRE && FMT != FMT_F16) {
    if (pl.mh == 2) {   // M = 9..16 on 8-row tiles: twelve waves (the activations are large)
      if (pl.nw == kNWBig) return launch5<FMT, EPI, RPW, PRE, kNWBig, 2>(k, pl, s);
      return hipErrorInvalidValue;
    }
  }
  if (pl.mh != 1) return hipErrorInvalidValue;
  // (int8 with the pre-norm always takes twelve waves: its eight-wave build
  // spills registers)
  if constexpr (!(FMT == FMT_INT8 && PRE)) {
    if (pl.nw == kNWSmall) return launch5<FMT, EPI, RPW, PRE, kNWSmall, 1>(k, pl, s);
  }
  if (pl.nw == kNWBig) return launch5<FMT, EPI, RPW, PRE, kNWBig, 1>(k, pl, s);
  return hipErrorInvalidValue;
}

template <int FMT, int EPI, int RPW>
hipError_t launch3(const RowsKArgs& k, const RowsPlan& pl, hipStream_t s) {
  if constexpr (FMT != FMT_F16) {
    if (k.pre_weight) return launch4<FMT, EPI, RPW, true>(k, pl, s);
  }
  return launch4<FMT, EPI, RPW, false>(k, pl, s);
}

template <int FMT, int EPI>
hipError_t launch2(const RowsKArgs& k, const RowsPlan& pl, hipStream_t s) {
  switch (pl.rpw) {
    case 1: return EPI == EPI_SWIGLU ? hipErrorInvalidValue : launch3<FMT, EPI, 1>(k, pl, s);
    case 2: return launch3<FMT, EPI, 2>(k, pl, s);
    case 4: return launch3<FMT, EPI, 4>(k, pl, s);
    case 8:   // 8-row tiles: 2 K shifts, quantized formats only (an fp16 step would be 64 k)
      if constexpr (FMT != FMT_F16) return launch3<FMT, EPI, 8>(k, pl, s);
      return hipErrorInvalidValue;
    case 16:   // 16-row tiles, no K shift: M = 9..16, quantized formats only
      if constexpr (FMT != FMT_F16) return launch3<FMT, EPI, 16>(k, pl, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <int FMT>
hipError_t launch1(const RowsKArgs& k, const RowsPlan& pl, int epi, hipStream_t s) {
  if (FMT == FMT_F16 || epi != EPI_SWIGLU) return launch2<FMT, EPI_NONE>(k, pl, s);
  return launch2<FMT, EPI_SWIGLU>(k, pl, s);
}

int kpl_of(int fmt) { return fmt == FMT_INT4 ? 32 : (fmt == FMT_INT8 ? 16 : 8); }
size_t al16(size_t v) { return (v + 15) & ~(size_t)15; }
int gshift_of(const LinearArgs& a) {
  if (a.fmt == FMT_F16 || a.G == 1) return 31;
  for (int b = 0; b < 31; ++b)
    if (a.g == (1 << b)) return b;
  return -1;
}
int xswz_h(int k) { return k + ((k >> 7) << 3); }

}  // namespace

namespace {

RowsPlan rows_plan_k(const LinearArgs& a, int num_cus, int KP) {
  RowsPlan p{};
  p.ok = false;
  const int kpl = kpl_of(a.fmt);
  if (a.M < 1 || a.M > (a.fmt == FMT_F16 ? 4 : 16)) return p;
  if (a.K % kpl != 0 || (a.K & 7)) return p;
  if (a.fmt != FMT_F16 && a.G != 1 && (gshift_of(a) < 0 || a.g < kpl)) return p;
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return p;
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return p;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return p;
  const int64_t lim = (int64_t)1 << 31;
  if (((int64_t)(a.M - 1) * a.lda + a.K) * 2 >= lim) return p;
  if ((int64_t)a.N * a.G * 2 >= lim) return p;
  const bool quant = a.fmt != FMT_F16;
  const int nrows = a.epi == EPI_SWIGLU ? a.F : a.N;
  // the tile width (>= M rows) with the least padded work per CU: rows per
  // workgroup rounded up to whole tiles, times K rounded up to whole steps,
  // for M = 1 less 3 % per doubling of the tile width (measured, int4,
  // K = 3584: 4 or 8 rows per tile 3-5 % faster than 1 or 2 at equal padded
  // work; K = 18944: 2 and 8 equal), otherwise 1 % more per row of width
  // (config 2 at M = 4: 4-row tiles 4 % faster than 8-row ones)
  int rpw = 4;
  double best_work = 1e300;
  for (int cand = 1; cand <= (a.fmt == FMT_F16 ? 4 : 16); cand <<= 1) {
    if (cand < a.M || (a.epi == EPI_SWIGLU && cand < 2) || (cand == 16 && a.M <= 8)) continue;
    const int ks = 4 * kpl * (16 / cand);
    const int gr = a.epi == EPI_SWIGLU ? cand / 2 : cand;
    const int rr = ((nrows + num_cus - 1) / num_cus + gr - 1) / gr * gr;
    const double pref = a.M == 1 ? 1.0 - 0.03 * __builtin_ctz(cand) : 1.0 + 0.01 * cand;
    const double work = (double)rr * ((a.K + ks - 1) / ks * ks) * pref;
    if (work < best_work) { best_work = work; rpw = cand; }
  }
  // M = 9..16 (quantized, no pre-norm): 8-row tiles with the activation rows
  // in two halves (two MFMAs per dequantized fragment) instead of 16-row
  // tiles, whose per-lane loads cover 64 bytes of each of 16 rows
  int mh = 1;
#ifndef MQ_ROWS_NO_MH2
  if (quant && !a.prenorm && a.M >= 9 && a.M <= 16) {
    rpw = 8;
    mh = 2;
  }
#endif
  const int S = 16 / rpw;
  const int kstep = 4 * kpl * S;
  const int gran = a.epi == EPI_SWIGLU ? rpw / 2 : rpw;  // output rows per tile
  // rows per workgroup: a whole number of tiles, one workgroup (one K part
  // of a row block) per CU
  int R = (int)(((int64_t)nrows * KP + num_cus - 1) / num_cus);
  R = (R + gran - 1) / gran * gran;
  const int nblk = (nrows + R - 1) / R;
  const int nwg = nblk * KP;
  const int TW = R / gran;
  const int KStot = (a.K + kstep - 1) / kstep;
  const int KS = (KStot + KP - 1) / KP;   // steps per part
  if (KP > 1 && (int64_t)KS * (KP - 1) >= KStot) return p;   // every part has steps
  const int U = TW * KS;
  const int64_t wbytes = (int64_t)(a.epi == EPI_SWIGLU ? 2 * R : R) * a.ldw / KP;   // weight bytes per workgroup
  const int nw = mh == 2 || wbytes > kSmallBytes || (a.prenorm && a.fmt == FMT_INT8) ? kNWBig : kNWSmall;
  const int per = (U + nw - 1) / nw;
  const int maxT = per / KS + 2;
  if ((int64_t)(a.epi == EPI_SWIGLU ? a.F + R : R) * a.ldw >= lim) return p;
  int XS = xswz_h(KS * kstep) + 8;
  // the LDS row stride of A (mod 256 bytes): 128 bytes for tiles with K
  // shifts; 16 bytes for 16-row tiles, whose 16 fragment rows (one per lane
  // of a 16-lane group) then fall in different banks
  XS = (XS + 127) / 128 * 128 + (rpw == 16 ? 8 : 64);
  size_t off = al16((size_t)a.M * XS * 2);
  p.off_sz = (uint32_t)off;
  // steps past K read up to kstep / g entries beyond a row's last group; a
  // region starts up to 7 entries below its first row's
  const int szpad = quant && a.G != 1 ? kstep / a.g + 1 : 0;
  if (quant && a.G != 1 && kstep % a.g != 0) return p;   // the scale entry advances by whole groups per step
  const int64_t snp = quant ? (7 + (int64_t)R * a.G + szpad + 7) / 8 : 0;
  const int nreg = a.epi == EPI_SWIGLU ? 2 : 1;
  if (snp * nreg * 32 > (int64_t)kLds) return p;
  off += (size_t)(snp * nreg * 32);
  p.off_scr = (uint32_t)off;
  off += (size_t)nw * 256 * 4;
  p.off_slot = (uint32_t)off;
  off += al16((size_t)nw * maxT * a.M * rpw * 4);
  p.off_wft = (uint32_t)off;
  off += al16((size_t)nw * 4);
  if (off > kLds) return p;
  if ((int64_t)U * nw >= ((int64_t)1 << 31)) return p;  // unit ranges in 32-bit arithmetic
  if (a.prenorm) {  // one staging batch, whole 16-byte pieces, M = 1
    const int64_t pieces = (int64_t)KS * kstep / 8;
    if (a.M != 1 || !quant || a.K % 8 || pieces > (int64_t)kXB * 64 * nw || !a.pre_weight || !a.pre_resid) return p;
    if (((uintptr_t)a.pre_weight | (uintptr_t)a.pre_resid | (uintptr_t)a.pre_delta) & 15) return p;
  }
  p.rpw = rpw; p.mh = mh; p.nw = nw; p.nwg = nwg; p.R = R; p.TW = TW; p.KS = KS; p.XS = XS; p.maxT = maxT;
  p.KP = KP; p.nblk = nblk; p.KStot = KStot;
  p.ws_bytes = KP > 1 ? kCntBytesRows + (size_t)KP * nblk * a.M * R * (a.epi == EPI_SWIGLU ? 2 : 1) * 4 : 0;
  if (KP > 1 && (size_t)nblk * 4 > kCntBytesRows) return p;
  p.snp = (int)snp;
  p.lds_bytes = off;
  p.ok = true;
  return p;
}

}  // namespace

RowsPlan rows_plan(const LinearArgs& a, int num_cus, bool allow_split) {
  RowsPlan p{};
  p.ok = false;
  // K parts: the fewest whose activation slice fits in LDS (more rows per
  // workgroup, so that the parts of all row blocks still cover the CUs once)
  for (int kp = 1; kp <= (allow_split && !a.prenorm ? 4 : 1); ++kp) {
    p = rows_plan_k(a, num_cus, kp);
    if (p.ok) return p;
  }
  return p;
}

hipError_t rows_launch(const LinearArgs& a, const RowsPlan& pl, void* ws, hipStream_t s) {
  if (!pl.ok) return hipErrorInvalidValue;
  if (pl.KP > 1 && !ws) return hipErrorInvalidValue;
  RowsKArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.ep = a.epi_args();
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.K = a.K; k.N = a.N; k.F = a.F; k.G = a.G;
  k.gshift = gshift_of(a);
  k.KStot = pl.KStot; k.KP = pl.KP; k.nblk = pl.nblk;
  if (pl.KP > 1) {
    k.cnt = (uint32_t*)ws;
    k.part = (float*)((char*)ws + kCntBytesRows);
  }
  k.R = pl.R; k.TW = pl.TW; k.KS = pl.KS; k.XS = pl.XS; k.maxT = pl.maxT; k.snp = pl.snp;
  k.off_sz = pl.off_sz; k.off_scr = pl.off_scr; k.off_slot = pl.off_slot; k.off_wft = pl.off_wft;
  if (a.prenorm) {
    k.pre_delta = (const _Float16*)a.pre_delta;
    k.pre_weight = (const _Float16*)a.pre_weight;
    k.pre_resid = (_Float16*)a.pre_resid;
    k.pre_eps = a.pre_eps;
  }
  k.sz_bytes = a.fmt == FMT_F16 ? 0u : (uint32_t)(((int64_t)a.N * a.G * 2 + 3) & ~(int64_t)3);
  k.z_bytes = a.zeros ? k.sz_bytes : 0u;
  switch (a.fmt) {
    case FMT_INT4: return launch1<FMT_INT4>(k, pl, a.epi, s);
    case FMT_INT8: return launch1<FMT_INT8>(k, pl, a.epi, s);
    default: return launch1<FMT_F16>(k, pl, a.epi, s);
  }
}

}  // namespace mq
