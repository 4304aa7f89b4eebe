// Prefill dequant GEMM (int4 and int8 weights, M-heavy shapes): C =
// epi(A . deq(W)^T), fp16 products accumulated in fp32 by
// v_mfma_f32_16x16x32_f16, one rounding.  Its main cases: the Llama-3.2-3B
// fused-QKV shape at M = 512 (int4, 128 x 80 tiles) and the Qwen2.5-7B
// gate/up shape at M = 64 with the SwiGLU epilogue (int8 per-channel,
// 64-row tiles of 80 gate + 80 up weight columns, 80 output columns).
//
// Replaces dequant_matmul_int4_fp16 / dequant_matmul_int8_fp16
// (shaders/matmul_dequant_kernel.metal:55-223, :351-479; dispatched at
// src/ops/matmul.mm:1011-1021), with the fused epilogues of
// shaders/matmul_fused_epilogue.metal:97-124 and the SwiGLU of
// shaders/fused_swiglu.metal:48-84.
//
// Structure:
//  * Workgroup = 4 waves (one per SIMD) on one output tile of 16*MBK rows by
//    16*NB weight columns.  Wave w takes every fourth 64-k K-tile from the
//    w-th, so every weight is loaded and dequantized once per workgroup and
//    every activation moved once.
//  * Activations: direct-to-LDS 16-byte loads (buffer_load ... lds), fully
//    coalesced, in a ring of 2 slots per wave (16 KiB for 128-row tiles,
//    8 KiB for 64-row tiles; 32 KiB per wave in all, the rest used by the
//    partial exchange), XOR-swizzled so that the fragment reads (one row per
//    lane) are bank-conflict free.  A K-tile's second k-step fragments are
//    read first, so its slot is refilled (the wave's K-tile after next)
//    while its first k-step computes.
//  * Weights: lane (c, q) of block j loads the 16 k at 64t + 16q of its
//    column (8 bytes int4, 16 bytes int8): the first half is its B operand
//    of the tile's first k-step, the second half of the second (k-step s
//    covers k = 16q + 8s .. +7 for lane group q; the activation fragment of
//    the same lane reads the same k range).  Dequantized in registers with
//    the exact two-rounding formula; scales and zeros come from an LDS table
//    (s | z << 16) of the tile's weight rows, loaded before anything else.
//  * The inner loop is hand-ordered with volatile inline asm: each k-step
//    issues its MBK*NB MFMAs one at a time, each followed by a share of the
//    VALU ops that dequantize the next k-step's weights and by a share of
//    the next k-step's fragment reads and of the refill loads.  One wave per
//    SIMD issues in order, so MFMA and VALU overlap only when interleaved;
//    the compiler's own schedule clusters them (and its register allocator
//    rotates the accumulators between AGPRs when it picks the untied MFMA
//    form), hence the asm with tied "+a" accumulators.  The weights are the
//    MFMA's first operand: each lane's accumulator then holds four adjacent
//    output columns of one row.
//  * After the K loop each wave writes the partials of the blocks it does
//    not own into its own activation slots; after one barrier the owner of
//    an output unit (a block; with SwiGLU a gate block and its up block)
//    sums the four partials in wave order (deterministic), applies the
//    epilogue to the fp32 sums, and the fp16 results are staged in LDS and
//    written back with 16-byte stores.
//
// Hazards of the inline-asm MFMAs (the compiler does not see inside them):
// every VGPR an MFMA reads was written by VALU at least one full region of
// MFMAs earlier or by an LDS read that the compiler waits for; each
// accumulator is only read and written by MFMAs of the same shape until the
// read-out, which is preceded by 24 wait states.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <algorithm>
#include <type_traits>

namespace mq {
namespace {

constexpr int G16_KT = 64;       // k per K-tile
constexpr int G16_SZT = 8192;    // scale|zero table entries (32 KiB)
constexpr int G16_AU = 2048;     // activation space per wave: 2048 16-byte pieces (32 KiB)

struct G16Args {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros;
  EpiArgs ep;
  _Float16* C; int64_t ldc;
  int M, N, K, G, gshift;
  int F;              // output columns: N/2 with SwiGLU, else N
  int nbm, KT, xcd;
  int SG;             // scale|zero table row stride: G + 1 rounded up to odd (column G is zero)
  Div32 gdiv;         // division by G
  int vec_store;      // C rows 16-byte aligned: staged 16-byte stores
  uint32_t a_bytes, w_bytes, s_bytes;
  uint64_t* trace;    // optional per-wave timestamps (tests of the schedule only)
};

__device__ __forceinline__ void dma16(rsrc_t r, u4* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

typedef uint32_t u2v __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// Activation slot I of the four waves: a separate LDS array per slot, so
// that the compiler's load-counter waits tell one slot's loads from another's.
template <int I, int S>
__device__ __forceinline__ u4 (&g16_slot())[4][S] {
  __shared__ u4 a[4][S];
  return a;
}

// Output units: blocks (i, j) with j < NBU; with SwiGLU block j + NBU (its up
// block) belongs to the unit of block j.  Unit i*NBU + j is owned by wave
// (i*NBU + j) % 4.
template <int NB, bool SWI>
__host__ __device__ constexpr int g16_owner(int i, int j) {
  constexpr int NBU = SWI ? NB / 2 : NB;
  return (i * NBU + j % NBU) % 4;
}
// position of block (i, j) among the blocks that wave ww does not own
template <int NB, bool SWI>
__host__ __device__ constexpr int g16_rank(int ww, int i, int j) {
  int r = 0;
  for (int b = 0; b < i * NB + j; ++b)
    if (g16_owner<NB, SWI>(b / NB, b % NB) != ww) ++r;
  return r;
}

template <int FMT, int MBK, int NB, bool SWI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm16_kernel(G16Args p) {
  // weight ring depth in K-tiles: 2 (with a 4-deep ring the int4 kernel
  // measured 1.5-3 % slower at config 3, g = 128 / 64 / 32)
  constexpr int WPF = 2;
  constexpr int NBU = SWI ? NB / 2 : NB;        // output blocks per row block
  constexpr int BNO = 16 * NBU;                 // output columns per tile
  constexpr int BM = 16 * MBK;                  // rows per tile
  constexpr int SLOTU = BM * 8;                 // 16-byte pieces per activation slot (BM rows x 64 k)
  constexpr int NS = G16_AU / SLOTU;            // 16-byte slots of the wave's activation space
  // activation ring depth: 2 slots (one K-tile of lead beyond the current);
  // with the 2-deep weight ring the K-tile loop is unrolled by 2 (static ring
  // indices), so a wave's last K-tiles fill the unroll (int8: 14 K-tiles per
  // wave at config 4, which a 4-tile unroll would round up to 16)
  constexpr int NSA = 2;
  constexpr int UNR = 2;                        // K-tiles per loop iteration
  constexpr int NDMA = 2 * MBK;                 // DMA instructions per K-tile (8 rows each)
  constexpr int WB = FMT == FMT_INT4 ? 8 : 16;  // weight bytes per lane per K-tile
  constexpr int NRANGE = SWI ? 2 : 1;           // weight row ranges (gate, up)
  static_assert(NS == 2 || NS == 4, "the activation space is 2 or 4 slots");
  static_assert(NSA <= NS && WPF == UNR && NSA == UNR, "the rings rotate with the 2-tile unroll");
  static_assert(!SWI || NB % 2 == 0, "SwiGLU pairs gate and up blocks");
  static_assert(MBK * NB - (MBK * NB) / 4 <= 32, "a wave's partials fit in its activation space");
  typedef typename std::conditional<FMT == FMT_INT4, u2v, u4>::type WReg;
  // scale | zero << 16 of the tile's weight rows x all groups, rows SG apart
  // (odd: the 16 rows one read touches fall in different banks), column G
  // zero (read by K-tiles past the wave's range)
  __shared__ uint32_t lds_sz[G16_SZT];
  const uint64_t T0 = __builtin_amdgcn_s_memrealtime();
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, q = lane >> 4;
  int id = blockIdx.x;
  if (p.xcd) {   // workgroup i runs on XCD i % 8: give each XCD a contiguous run of tiles
    const int per = gridDim.x >> 3;
    id = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  }
  const int nb = id / p.nbm, mb = id - nb * p.nbm;   // M-block fastest: neighbours share weights
  const int m0 = mb * BM, n0 = nb * BNO;             // first row, first output column
  const rsrc_t ar = make_rsrc(p.A, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  const rsrc_t sr = make_rsrc(p.scales, p.s_bytes);
  const rsrc_t zr = make_rsrc(p.zeros, p.s_bytes);
  const rsrc_t nullr = make_rsrc(p.A, 0);   // every load through it reads zeros
  // wave w takes K-tiles w, w + 4, w + 8, ...: the four waves read
  // neighbouring 64-k pieces of the same activation and weight rows at once
  // (contiguous quarters of K measured 1-3.5 % slower at configs 3 and 4)
  constexpr int TS = 4;   // K-tile stride of a wave
  const int kt0 = w, kt1 = p.KT;
  const int ncols = min(BNO, p.F - n0);     // real output columns of the tile

  // ---- scale | zero table, first: per weight row range (the tile's
  // columns; with SwiGLU their gate rows, then their up rows F below) the
  // [G] entries of each row, as 16-byte pieces of the [N, G] arrays, every
  // load issued before the first LDS write ----
  const int cnt = ncols * p.G;                 // entries per range
  const uint32_t sreal = (uint32_t)p.N * (uint32_t)p.G * 2u;
  constexpr int SPT = 4;                       // pieces per thread and range (<= 8184 entries)
  u4 sv[NRANGE][SPT], zv[NRANGE][SPT];
#pragma unroll
  for (int rg = 0; rg < NRANGE; ++rg) {
    const int e0 = (rg ? p.F + n0 : n0) * p.G;
    const int pb = e0 >> 3, pe = (e0 + cnt + 7) >> 3;
#pragma unroll
    for (int r = 0; r < SPT; ++r) {
      sv[rg][r] = zv[rg][r] = (u4){0u, 0u, 0u, 0u};
      if (pb + 256 * r >= pe) continue;   // no lane of the workgroup has a piece
      const int pc = pb + tid + 256 * r;
      const uint32_t off = (uint32_t)pc * 16u;
      const bool ok = pc < pe && off + 16u <= sreal;
      sv[rg][r] = bload16(sr, ok ? off : kOob);
      zv[rg][r] = bload16(zr, ok ? off : kOob);
    }
  }

  // ---- activations: DMA instruction i moves rows 8i..8i+7 of the K-tile;
  // lane l -> row 8i + l/8, LDS position l%8, k-piece (l%8) ^ (row%8) ----
  const int pa = (lane & 7) ^ (lane >> 3);
  const uint32_t rstride = (uint32_t)(8 * p.lda * 2);
  // MFMA fragment of row block i, k-step s: row 16i + c, k-piece 2q + s
  uint32_t ard[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) ard[s] = (uint32_t)(c * 8 + ((2 * q + s) ^ (c & 7)));

  // ---- weights: block j, lane c is weight row n0 + 16j + c (SwiGLU: the
  // blocks from NB/2 on are the up rows F + n0 + 16(j - NB/2) + c) ----
  uint32_t woff[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int lo = 16 * (j % NBU) + c;   // output column within the tile
    const int row = (SWI && j >= NBU ? p.F : 0) + n0 + lo;
    woff[j] = lo < ncols ? (uint32_t)(row * p.ldw) + (uint32_t)(WB * q) : kOob;
  }
  WReg wring[WPF][NB];
  auto load_w = [&](int t, WReg (&dst)[NB]) {
    const bool past = t >= kt1;
    const uint32_t so = past ? 0u : (uint32_t)t * (uint32_t)(4 * WB);
    const rsrc_t rr = past ? nullr : wr;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if constexpr (FMT == FMT_INT4)
        dst[j] = __builtin_bit_cast(WReg, __builtin_amdgcn_raw_buffer_load_b64(rr, woff[j], so, 0));
      else
        dst[j] = __builtin_bit_cast(WReg, __builtin_amdgcn_raw_buffer_load_b128(rr, woff[j], so, 0));
    }
  };

  auto slot = [&](auto ac) -> u4* { return g16_slot<decltype(ac)::value, SLOTU>()[w]; };
  // Activations: one lane offset (row m0 + l/8, piece pa); row group i adds
  // i*8 rows through the scalar offset.  The buffer's range ends with row
  // M-1 and the range check includes the scalar offset, so rows past M read
  // zeros (they only reach output rows that are never stored).
  const uint32_t adma = (uint32_t)((m0 + (lane >> 3)) * p.lda * 2) + 16u * pa;
  auto dma_one = [&](int t, u4* sl, int i) {
    const bool past = t >= kt1;
    const uint32_t so = past ? 0u : (uint32_t)t * 128u;
    dma16(past ? nullr : ar, sl + 64 * i, adma, so + i * rstride);
  };
  auto dma_tile = [&](int t, u4* sl) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma_one(t, sl, i);
  };
  // prologue loads: what the first K-tile's k-step 0 needs (its activations
  // and weights) and the next K-tile's weights; the rest of the pipeline's
  // loads go out when the first K-tile starts (a deep burst issued here
  // would hold back the first data: every CU starts at once)
  dma_tile(kt0, slot(std::integral_constant<int, 0>{}));
  load_w(kt0, wring[0]);
  load_w(kt0 + TS, wring[1]);
  // scale | zero table writes (s | z << 16 per entry; range rg from row
  // rg * BNO), then the zero column
  const int SG = p.SG;
#pragma unroll
  for (int rg = 0; rg < NRANGE; ++rg) {
    const int e0 = (rg ? p.F + n0 : n0) * p.G;
    const int d0 = rg * BNO * SG;
    const int pb = e0 >> 3, pe = (e0 + cnt + 7) >> 3;
#pragma unroll
    for (int r = 0; r < SPT; ++r) {
      const int pc = pb + tid + 256 * r;
      if (pc >= pe) break;
      const uint32_t off = (uint32_t)pc * 16u;
      uint32_t sw[4] = {sv[rg][r].x, sv[rg][r].y, sv[rg][r].z, sv[rg][r].w};
      uint32_t zw[4] = {zv[rg][r].x, zv[rg][r].y, zv[rg][r].z, zv[rg][r].w};
      if (off + 16u > sreal) {   // the piece that straddles the end of the arrays: entry by entry
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t o0 = off + 4u * e, o1 = o0 + 2u;
          sw[e] = bload2(sr, o0 < sreal ? o0 : kOob) | (bload2(sr, o1 < sreal ? o1 : kOob) << 16);
          zw[e] = bload2(zr, o0 < sreal ? o0 : kOob) | (bload2(zr, o1 < sreal ? o1 : kOob) << 16);
        }
      }
      // entry le of the range is (row, group) = (le / G, le % G): the first
      // entry's by one division, the rest by stepping (entries below 0 are
      // skipped and keep row 0)
      const int lb = pc * 8 - e0;
      int row = lb > 0 ? (int)p.gdiv.div((uint32_t)lb) : 0;
      int col = lb - row * p.G;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int le = lb + e;
        if (le >= 0 && le < cnt)
          lds_sz[d0 + row * SG + col] =
              ((sw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) | ((zw[e >> 1] >> (16 * (e & 1))) << 16);
        if (++col == p.G) { col = 0; ++row; }
      }
    }
  }
  if (tid < NRANGE * BNO) lds_sz[tid * SG + p.G] = 0u;
  __syncthreads();
  const uint64_t T1 = __builtin_amdgcn_s_memrealtime();

  // scale|zero of K-tile t for each block; K-tiles past the wave's range
  // get (0, 0), so their (zero) activations meet zero weights.  Block j's
  // lane c is table row 16j + c (SwiGLU: up rows from BNO on).
  const int szrow = c * SG;
  auto read_sz = [&](int t, uint32_t (&dst)[NB]) {
    const int g = t >= kt1 ? p.G : p.gshift >= 31 ? 0 : min((t * 64 + 16 * q) >> p.gshift, p.G - 1);
#pragma unroll
    for (int j = 0; j < NB; ++j) dst[j] = lds_sz[szrow + 16 * j * SG + g];
  };

  f4 acc[MBK][NB];
#pragma unroll
  for (int i = 0; i < MBK; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

  // dequant constants (a VOP3 takes one scalar operand: the others in VGPRs)
  uint32_t nmask = 0x00F0000Fu, fo = 0xD480E408u, c64 = 0x64646464u;
  asm volatile("" : "+v"(nmask), "+v"(fo), "+v"(c64));
  const uint32_t magic = 0x64006400u;
  const uint32_t sel0 = 0x0c000c00u, sel1 = 0x0c010c01u, sel2 = 0x0c020c02u, sel3 = 0x0c030c03u;
  const uint32_t fm = 0x2C003C00u;                           // fp16 pair (1, 1/16)
  const uint32_t b8lo = 0x04010400u, b8hi = 0x04030402u;     // int8: bytes 0,1 / 2,3 under 0x64
  const uint32_t m1152 = 0xE480E480u;                        // fp16 pair (-1152, -1152)

  // One k-step, hand-ordered: region j (weight block j) issues the MBK MFMAs
  // of (bq[j], af[i]) one by one, each followed by a share of the VALU ops
  // that dequantize block j of the next k-step, and by a share of the next
  // k-step's fragment reads and of `extra` (refill loads).  EARLY: all of the
  // next k-step's fragments are read at the start (their slot can then be
  // refilled during this k-step).
  auto step = [&](auto earlyc, const h8 (&af)[MBK], const h8 (&bq)[NB], const u4* nsl, int ns, h8 (&naf)[MBK],
                  const WReg (&nwt)[NB], const uint32_t (&nsz)[NB], int nstep, h8 (&nbq)[NB], auto extra) {
    constexpr bool EARLY = decltype(earlyc)::value;
    if (EARLY) {
#pragma unroll
      for (int i = 0; i < MBK; ++i) naf[i] = __builtin_bit_cast(h8, nsl[ard[ns] + 128 * i]);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const uint32_t e = nsz[j];
      uint32_t x0, x1, x2, x3;
#define MF(i) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc[i][j]) : "v"(bq[j]), "v"(af[i]))
#define MUL(x) asm volatile("v_pk_mul_f16 %0, %1, %0 op_sel_hi:[0,1]" : "+v"(x) : "v"(e))
#define SUB(x) asm volatile("v_pk_add_f16 %0, %0, %1 op_sel:[0,1] neg_lo:[0,1] neg_hi:[0,1]" : "+v"(x) : "v"(e))
#define SB() __builtin_amdgcn_sched_barrier(0)
#define NAF(r)                                                                                 \
  if (!EARLY && (j * MBK) / NB + (r) < ((j + 1) * MBK) / NB)                                   \
    naf[(j * MBK) / NB + (r)] = __builtin_bit_cast(h8, nsl[ard[ns] + 128 * ((j * MBK) / NB + (r))]);
      if constexpr (FMT == FMT_INT4) {
        // k0..k7 of one dword: each pair's byte under 0x6400 (1024 + lo,
        // 1024 + 16 hi), one packed FMA to (lo - 8, hi - 8) exactly, then
        // RNE(q*s) and RNE(. - z): the reference's two roundings
        static_assert(MBK == 8, "the int4 schedule spreads a block's dequant over 8 MFMAs");
        const uint32_t d = nstep ? nwt[j][1] : nwt[j][0];
#define PERM(x, sel) asm volatile("v_perm_b32 %0, 0, %1, %2" : "=v"(x) : "v"(d), "s"(sel))
#define ANDOR(x) asm volatile("v_and_or_b32 %0, %0, %1, %2" : "+v"(x) : "v"(nmask), "s"(magic))
#define FMA(x) asm volatile("v_pk_fma_f16 %0, %0, %1, %2" : "+v"(x) : "s"(fm), "v"(fo))
        MF(0); PERM(x0, sel0); PERM(x1, sel1); ANDOR(x0); SB();
        MF(1); PERM(x2, sel2); PERM(x3, sel3); ANDOR(x1); SB();
        NAF(0)
        SB();
        MF(2); ANDOR(x2); ANDOR(x3); FMA(x0); SB();
        MF(3); FMA(x1); FMA(x2); FMA(x3); SB();
        NAF(1)
        extra(j);
        SB();
        MF(4); MUL(x0); MUL(x1); SUB(x0); SB();
        MF(5); MUL(x2); MUL(x3); SUB(x1); SB();
        MF(6); SUB(x2); SB();
        MF(7); SUB(x3); SB();
#undef PERM
#undef ANDOR
#undef FMA
      } else {
        // four int8 of one dword: XOR 0x80 makes them q+128 (0..255); two
        // bytes under 0x64 are 1152 + q exactly; minus 1152 (exact); then
        // RNE(q*s) and RNE(. - z)
        static_assert(MBK == 4 || MBK == 8, "int8 schedules for 4 and 8 row blocks");
        const uint32_t d0 = nstep ? nwt[j][2] : nwt[j][0], d1 = nstep ? nwt[j][3] : nwt[j][1];
        uint32_t u0, u1;
#define XOR(u, d) asm volatile("v_xor_b32 %0, 0x80808080, %1" : "=v"(u) : "v"(d))
#define PERM8(x, u, sel) asm volatile("v_perm_b32 %0, %1, %2, %3" : "=v"(x) : "v"(c64), "v"(u), "s"(sel))
#define SUB8(x) asm volatile("v_pk_add_f16 %0, %0, %1" : "+v"(x) : "s"(m1152))
        if constexpr (MBK == 4) {
          MF(0); XOR(u0, d0); XOR(u1, d1); PERM8(x0, u0, b8lo); PERM8(x1, u0, b8hi); PERM8(x2, u1, b8lo); SB();
          NAF(0)
          extra(j);
          SB();
          MF(1); PERM8(x3, u1, b8hi); SUB8(x0); SUB8(x1); SUB8(x2); SUB8(x3); SB();
          MF(2); MUL(x0); MUL(x1); MUL(x2); MUL(x3); SB();
          MF(3); SUB(x0); SUB(x1); SUB(x2); SUB(x3); SB();
        } else {
          MF(0); XOR(u0, d0); XOR(u1, d1); PERM8(x0, u0, b8lo); SB();
          MF(1); PERM8(x1, u0, b8hi); PERM8(x2, u1, b8lo); PERM8(x3, u1, b8hi); SB();
          NAF(0)
          SB();
          MF(2); SUB8(x0); SUB8(x1); SUB8(x2); SB();
          MF(3); SUB8(x3); MUL(x0); MUL(x1); SB();
          NAF(1)
          extra(j);
          SB();
          MF(4); MUL(x2); MUL(x3); SB();
          MF(5); SUB(x0); SUB(x1); SB();
          MF(6); SUB(x2); SB();
          MF(7); SUB(x3); SB();
        }
#undef XOR
#undef PERM8
#undef SUB8
      }
      u4 o;
      o.x = x0; o.y = x1; o.z = x2; o.w = x3;
      nbq[j] = __builtin_bit_cast(h8, o);
#undef MF
#undef MUL
#undef SUB
#undef SB
#undef NAF
    }
  };

  // first k-step's operands (C++ dequant; outside the loop)
  h8 afA[MBK], afB[MBK], bqA[NB], bqB[NB];
  uint32_t sz[NB], sz2[NB];
#pragma unroll
  for (int i = 0; i < MBK; ++i) afA[i] = __builtin_bit_cast(h8, slot(std::integral_constant<int, 0>{})[ard[0] + 128 * i]);
  read_sz(kt0, sz);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const h2 e = as_h2(sz[j]);
    const h2 s2 = __builtin_shufflevector(e, e, 0, 0), z2 = __builtin_shufflevector(e, e, 1, 1);
    if constexpr (FMT == FMT_INT4) {
      bqA[j] = dq_int4_dword_nat_r(wring[0][j][0], s2, z2, nmask, magic);
    } else {
      h2 q0, q1, q2, q3;
      dq_int8_dword(wring[0][j][0], s2, z2, q0, q1);
      dq_int8_dword(wring[0][j][1], s2, z2, q2, q3);
      h8 b;
      b.s01 = q0; b.s23 = q1; b.s45 = q2; b.s67 = q3;
      bqA[j] = b;
    }
  }

  // the wave's K-tile t ((t - kt0) / TS = R mod UNR): activations in slot
  // R % NSA, weights in ring slot R % WPF; the wave's next K-tile (t + TS)
  // has its activations in slot (R+1) % NSA.
  auto tile = [&](auto rc, int t) {
    constexpr int R = decltype(rc)::value;
    constexpr int RW = R % WPF, RW1 = (R + 1) % WPF;
    u4* const cur = slot(std::integral_constant<int, R % NSA>{});
    u4* const nxt = slot(std::integral_constant<int, (R + 1) % NSA>{});
    if (R == 0 && t == kt0) {   // the first K-tile: the rest of the prologue
      dma_tile(kt0 + TS, slot(std::integral_constant<int, 1>{}));
    }
    read_sz(t + TS, sz2);
    // k-step 0 of tile t: reads all of k-step 1's fragments first; once
    // they are in registers the slot is refilled (K-tile t + NSA TS), spread over
    // the rest of the k-step; then the weight slot is refilled
    step(std::true_type{}, afA, bqA, cur, 1, afB, wring[RW], sz, 1, bqB, [&](int j) {
      if (j == 0) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int i = 0; i < NDMA; ++i)
        if ((i * NB) / NDMA == j) dma_one(t + NSA * TS, cur, i);
    });
    load_w(t + WPF * TS, wring[RW]);
    // k-step 1 of tile t; prepares tile t + TS's k-step 0 from slot `nxt`
    step(std::false_type{}, afB, bqB, nxt, 0, afA, wring[RW1], sz2, 0, bqA, [&](int) {});
#pragma unroll
    for (int j = 0; j < NB; ++j) sz[j] = sz2[j];
  };
  // two K-tiles per iteration (static ring indices: no register copies of
  // loads in flight); a K-tile past the wave's range reads zeros and has
  // zero scales
  int t = kt0;
  do {
    tile(std::integral_constant<int, 0>{}, t);
    tile(std::integral_constant<int, 1>{}, t + TS);
    t += UNR * TS;
  } while (t < kt1);
  const uint64_t T2 = __builtin_amdgcn_s_memrealtime();

  // ---- the four partial tiles meet in LDS ----
  // Each wave writes its partials of the blocks it does not own into its
  // own activation slots (free once its K loop is done: no barrier before),
  // 1 KiB per block in block order, 16 bytes per lane (conflict-free); after
  // one barrier each owner sums the four partials of its blocks in wave
  // order (deterministic).
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");   // MFMA results retired
#pragma unroll
  for (int i = 0; i < MBK; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) asm volatile("" : "+a"(acc[i][j]));
  // 1 KiB piece k of wave ww's activation space
  auto rslot = [&](int ww, int k) -> f4* {
    constexpr int per = SLOTU / 64;
    u4* base;
    if (k < per) base = g16_slot<0, SLOTU>()[ww];
    else if (k < 2 * per) base = g16_slot<1, SLOTU>()[ww];
    else if constexpr (NS > 2) base = k < 3 * per ? g16_slot<2 % NS, SLOTU>()[ww] : g16_slot<3 % NS, SLOTU>()[ww];
    else base = g16_slot<1, SLOTU>()[ww];   // (never: at most 2 * per pieces)
    return (f4*)base + (k % per) * 64;
  };
  constexpr int NU = MBK * NBU;           // output units
  constexpr int NOWN = (NU + 3) / 4;      // units per wave (at most)
  f4 own[NOWN][NRANGE];                   // fp32 sums of each owned unit (SwiGLU: gate, up)
  auto gather = [&](auto wc) {
    constexpr int W = decltype(wc)::value;
    // straight from the accumulator registers (no copies through VGPRs);
    // the 24 wait states above cover the MFMA-to-LDS-read dependency
#pragma unroll
    for (int i = 0; i < MBK; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        if (g16_owner<NB, SWI>(i, j) != W) {
          const uint32_t la =
              (uint32_t)(uintptr_t)(__attribute__((address_space(3))) f4*)(rslot(W, g16_rank<NB, SWI>(W, i, j)) + lane);
          asm volatile("ds_write_b128 %0, %1" :: "v"(la), "a"(acc[i][j]) : "memory");
        }
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();   // every wave's partials are in LDS
#pragma unroll
    for (int i = 0; i < MBK; ++i)
#pragma unroll
      for (int j = 0; j < NBU; ++j) {
        const int u = i * NBU + j;
        if (u % 4 != W) continue;
#pragma unroll
        for (int h = 0; h < NRANGE; ++h) {
          const int jj = j + h * NBU;
          f4 sum = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ww = 0; ww < 4; ++ww) {   // wave order: deterministic
            if (ww == W) sum += acc[i][jj];
            else sum += rslot(ww, g16_rank<NB, SWI>(ww, i, jj))[lane];
          }
          own[u >> 2][h] = sum;
        }
      }
  };
  if (w == 0) gather(std::integral_constant<int, 0>{});
  else if (w == 1) gather(std::integral_constant<int, 1>{});
  else if (w == 2) gather(std::integral_constant<int, 2>{});
  else gather(std::integral_constant<int, 3>{});
  __syncthreads();   // every partial has been read
  const uint64_t T4 = __builtin_amdgcn_s_memrealtime();
  // owned unit 4u + w: row block i, output block j; the lane holds row
  // 16i + c, output columns 16j + 4q .. +3
  auto unit_value = [&](int u, int v) -> float {
    if constexpr (SWI) return silu_f32((float)(_Float16)own[u][0][v]) * (float)(_Float16)own[u][NRANGE - 1][v];
    else return own[u][0][v];
  };
  u4* const stage = g16_slot<0, SLOTU>()[0];   // the first slot array of all four waves
  constexpr int PPR = BNO / 8;                  // 16-byte pieces per output row
  constexpr int NPC = (BM * PPR + 255) / 256;   // pieces per thread
  const int kind = p.ep.epi;
  if ((SWI || kind == EPI_NONE) && p.vec_store && m0 + BM <= p.M && ncols == BNO) {
    // fp16 results staged as [BM][SS] halves (rows 16 bytes apart mod 128
    // bytes: the 16 rows of one store group fall in different banks), then
    // 16-byte stores, every LDS read of a thread issued before its stores
    constexpr int SS = BNO + 8;
    _Float16* stg = (_Float16*)stage;
    static_assert(BM * SS * 2 <= 4 * SLOTU * 16, "output tile fits the first slot array");
#pragma unroll
    for (int u = 0; u < NOWN; ++u) {
      const int un = 4 * u + w;
      if (un >= NU) break;
      const int i = un / NBU, j = un - i * NBU;
      h4 hv;
#pragma unroll
      for (int v = 0; v < 4; ++v) hv[v] = (_Float16)unit_value(u, v);
      *(h4*)&stg[(16 * i + c) * SS + 16 * j + 4 * q] = hv;
    }
    __syncthreads();
    h8 pv[NPC];
#pragma unroll
    for (int e = 0; e < NPC; ++e) {
      const int pc = tid + 256 * e;
      const int r = pc / PPR, cc = 8 * (pc - r * PPR);
      if (pc < BM * PPR) pv[e] = *(const h8*)&stg[r * SS + cc];
    }
#pragma unroll
    for (int e = 0; e < NPC; ++e) {
      const int pc = tid + 256 * e;
      const int r = pc / PPR, cc = 8 * (pc - r * PPR);
      if (pc < BM * PPR) *(h8*)(p.C + (int64_t)(m0 + r) * p.ldc + n0 + cc) = pv[e];
    }
  } else {
    // fp32 values staged as [BM][RS] (SwiGLU: already combined); the
    // epilogue is applied per element, then fp16 rounding and 16-byte
    // stores where the rows allow
    constexpr int RS = BNO + 4;
    float* res = (float*)stage;
    static_assert(BM * RS * 4 <= 4 * SLOTU * 16, "result tile fits the first slot array");
#pragma unroll
    for (int u = 0; u < NOWN; ++u) {
      const int un = 4 * u + w;
      if (un >= NU) break;
      const int i = un / NBU, j = un - i * NBU;
      f4 v4;
#pragma unroll
      for (int v = 0; v < 4; ++v) v4[v] = unit_value(u, v);
      *(f4*)&res[(16 * i + c) * RS + 16 * j + 4 * q] = v4;
    }
    __syncthreads();
    for (int pc = tid; pc < BM * PPR; pc += 256) {
      const int r = pc / PPR, cc = 8 * (pc - r * PPR);
      const int row = m0 + r, col = n0 + cc;
      if (row >= p.M || cc >= ncols) continue;
      const f4 v0 = *(const f4*)&res[r * RS + cc], v1 = *(const f4*)&res[r * RS + cc + 4];
      float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      const int nc = min(8, ncols - cc);
      if (!SWI && kind != EPI_NONE) {
        for (int e = 0; e < nc; ++e) v[e] = epi_apply(v[e], (int64_t)row, col + e, p.ep);
      }
      _Float16* dst = p.C + (int64_t)row * p.ldc + col;
      if (p.vec_store && nc == 8) {
        h8 hv;
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[e] = (_Float16)v[e];
        *(h8*)dst = hv;
      } else {
        for (int e = 0; e < nc; ++e) dst[e] = (_Float16)v[e];
      }
    }
  }
  if (p.trace != nullptr && lane == 0) {
    uint64_t* o = p.trace + ((size_t)blockIdx.x * 4 + w) * 8;
    o[0] = T0; o[1] = T1; o[2] = T2; o[3] = T4; o[4] = __builtin_amdgcn_s_memrealtime();
  }
}

// Tile shapes: 128 rows x 80 columns; int8 SwiGLU up to M = 64: 64 rows x
// (80 gate + 80 up) weight columns.  SwiGLU with more than 64 rows is left
// to the other prefill kernels (its 128-row partials would not fit the
// activation space).
int g16_sg(int G) { return G + 1 + (G & 1); }

struct G16Shape {
  int mbk, nb;
  bool swi;
};

G16Shape pick(const LinearArgs& a) {
  const bool swi = a.epi == EPI_SWIGLU;
  if (a.fmt == FMT_INT8 && a.M <= 64 && swi) return {4, 10, true};
  return {8, 5, swi};
}

bool shape_ok(const LinearArgs& a) {
  if (a.fmt != FMT_INT4 && a.fmt != FMT_INT8) return false;
  if (a.prenorm) return false;
  if (a.M < 1 || a.N < 1 || a.K < 64 || a.K % 64 != 0) return false;
  const G16Shape sh = pick(a);
  if (sh.swi && (sh.mbk != 4 || a.N % 2 != 0 || a.F * 2 != a.N)) return false;
  if (a.lda % 8 != 0 || ((uintptr_t)a.A & 15) != 0) return false;     // 16-byte activation pieces
  const int wb = a.fmt == FMT_INT4 ? 8 : 16;                          // weight bytes per lane load
  if (a.ldw % wb != 0 || ((uintptr_t)a.W & (wb - 1)) != 0) return false;
  const bool per_channel = a.g >= a.K;
  if (!per_channel && (a.g < 16 || (a.g & (a.g - 1)) != 0)) return false;  // a lane's 16 k in one group
  // 32-bit buffer offsets
  if ((int64_t)a.M * a.lda * 2 >= (1ll << 31) || (int64_t)a.N * a.ldw >= (1ll << 31)) return false;
  if ((int64_t)a.N * a.G * 2 >= (1ll << 31)) return false;
  // scale|zero table: all weight rows of a tile (rows of g16_sg(G) entries), at
  // most 4 pieces per thread and range
  const int64_t range = (int64_t)(sh.swi ? 8 : 16) * sh.nb * a.G;
  const int64_t rows = (int64_t)(sh.swi ? 8 : 16) * sh.nb * (sh.swi ? 2 : 1);
  if (rows * g16_sg(a.G) > G16_SZT || range + 8 > 8 * 256 * 4) return false;
  return a.zeros != nullptr;
}

template <int FMT, int MBK, int NB, bool SWI>
void launch_one(const G16Args& k, int nwg, hipStream_t s) {
  hipLaunchKernelGGL((gemm16_kernel<FMT, MBK, NB, SWI>), dim3(nwg), dim3(256), 0, s, k);
}

}  // namespace

bool gemm16_supported(const LinearArgs& a) { return shape_ok(a); }

int gemm16_rows_per_tile(const LinearArgs& a) { return 16 * pick(a).mbk; }

int gemm16_workgroups(const LinearArgs& a) {
  const G16Shape sh = pick(a);
  const int bno = (sh.swi ? 8 : 16) * sh.nb;
  const int nout = sh.swi ? a.N / 2 : a.N;
  return ((a.M + 16 * sh.mbk - 1) / (16 * sh.mbk)) * ((nout + bno - 1) / bno);
}

hipError_t gemm16_launch(const LinearArgs& a, hipStream_t s, uint64_t* trace) {
  if (!shape_ok(a)) return hipErrorInvalidValue;
  const G16Shape sh = pick(a);
  G16Args k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.ep = a.epi_args();
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.G = a.G;
  k.F = sh.swi ? a.N / 2 : a.N;
  k.gshift = a.g >= a.K ? 31 : __builtin_ctz((unsigned)a.g);
  k.nbm = (a.M + 16 * sh.mbk - 1) / (16 * sh.mbk);
  k.KT = a.K / G16_KT;
  k.SG = g16_sg(a.G);
  k.gdiv = Div32::make((uint32_t)a.G);
  const int nwg = gemm16_workgroups(a);
  k.xcd = nwg % 8 == 0;
  k.vec_store = (a.ldc % 8 == 0) && (((uintptr_t)a.C & 15) == 0);
  // bytes of A up to the end of its last row, of W, of one scale array
  const int64_t wrow = a.fmt == FMT_INT4 ? a.K / 2 : a.K;
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  k.w_bytes = (uint32_t)((int64_t)(a.N - 1) * a.ldw + wrow);
  k.s_bytes = (uint32_t)((int64_t)a.N * a.G * 2);
  k.trace = trace;
  if (a.fmt == FMT_INT4) launch_one<FMT_INT4, 8, 5, false>(k, nwg, s);
  else if (sh.mbk == 4 && sh.swi) launch_one<FMT_INT8, 4, 10, true>(k, nwg, s);
  else launch_one<FMT_INT8, 8, 5, false>(k, nwg, s);
  return hipGetLastError();
}

}  // namespace mq
