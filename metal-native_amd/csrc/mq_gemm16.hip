// Prefill dequant GEMM for int4 weights, M-heavy shapes (the Llama-3.2-3B
// fused-QKV shape at M = 512 is its main case): C = epi(A . deq(W)^T), fp16
// products accumulated in fp32 by v_mfma_f32_16x16x32_f16, one rounding.
//
// Replaces dequant_matmul_int4_fp16 (shaders/matmul_dequant_kernel.metal:55-223,
// dispatched at src/ops/matmul.mm:1011-1021).
//
// Structure:
//  * Workgroup = 4 waves (one per SIMD) on one output tile of 128 rows by
//    16*NB columns (128 x 80 for NB = 5: 4 x 64 = 256 tiles at M = 512,
//    N = 5120, one per CU, and no MFMA spent on masked columns).  Wave w takes
//    the w-th quarter of the 64-k K-tiles, so every weight is loaded and
//    dequantized once per workgroup and every activation moved once.
//  * Activations: direct-to-LDS 16-byte loads (buffer_load ... lds), fully
//    coalesced, double-buffered per wave, XOR-swizzled so that the fragment
//    reads (one row per lane) are bank-conflict free.
//  * Weights: lane (c, q) of block j loads 8 bytes of column 16j + c at
//    k = 64t + 16q: its two dwords are exactly its B operands of the tile's
//    two k-steps (k-step s covers k = 16q + 8s .. +7 for lane group q; the
//    activation fragment of the same lane reads the same k range).
//    Dequantized in registers with the exact two-rounding formula; scales
//    and zeros come from an LDS table (s | z << 16) of the tile's columns,
//    loaded before anything else.
//  * The inner loop is hand-ordered with volatile inline asm: each k-step
//    issues its 40 MFMAs one at a time, each followed by two or three of the
//    VALU ops that dequantize the next k-step's weights and by a share of
//    the next k-step's fragment reads and of the refill loads.  One wave per
//    SIMD issues in order, so MFMA and VALU overlap only when interleaved;
//    the compiler's own schedule clusters them (and its register allocator
//    rotates the accumulators between AGPRs when it picks the untied MFMA
//    form), hence the asm with tied "+a" accumulators.
//  * After the K loop the four partial tiles meet in LDS (each wave owns a
//    quarter of the 16x16 blocks and sums the four partials in wave order,
//    deterministic), the epilogue is applied to the fp32 sums, the fp16
//    results are staged in LDS and written back with 16-byte stores.
//
// Hazards of the inline-asm MFMAs (the compiler does not see inside them):
// every VGPR an MFMA reads was written by VALU at least one full region
// (8 MFMAs) earlier or by an LDS read that the compiler waits for; each
// accumulator is only read and written by MFMAs of the same shape until the
// read-out, which is preceded by 24 wait states.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <algorithm>

namespace mq {
namespace {

constexpr int G16_KT = 64;       // k per K-tile
constexpr int G16_MB = 8;        // 16-row blocks per tile (128 rows)
constexpr int G16_SZT = 8192;    // scale|zero table entries (32 KiB)
constexpr int G16_WPF = 4;       // weight ring depth in K-tiles (loads issued up to 3 K-tiles ahead)

struct G16Args {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros;
  EpiArgs ep;
  _Float16* C; int64_t ldc;
  int M, N, K, G, gshift;
  int nbm, KT, xcd;
  int vec_store;      // C rows 16-byte aligned: staged 16-byte stores
  uint32_t a_bytes, w_bytes, s_bytes;
  uint64_t* trace;    // optional per-wave timestamps (tests of the schedule only)
};

__device__ __forceinline__ void dma16(rsrc_t r, u4* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

typedef uint32_t u2v __attribute__((ext_vector_type(2)));

template <int NB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm16_kernel(G16Args p) {
  constexpr int MBK = G16_MB;
  constexpr int WPF = G16_WPF;
  constexpr int BN = 16 * NB;
  static_assert(MBK * NB * 3 <= 128, "reduction slots must fit in the two activation arrays");
  __shared__ u4 lds_a0[4][1024];      // per wave: 128 rows x 64 k, slot 0
  __shared__ u4 lds_a1[4][1024];      // slot 1
  __shared__ uint32_t lds_sz[G16_SZT]; // scale | zero << 16 of the tile's columns x all groups
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
  const int m0 = mb * 128, n0 = nb * BN;
  const rsrc_t ar = make_rsrc(p.A, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  const rsrc_t sr = make_rsrc(p.scales, p.s_bytes);
  const rsrc_t zr = make_rsrc(p.zeros, p.s_bytes);
  const rsrc_t nullr = make_rsrc(p.A, 0);   // every load through it reads zeros
  const int kt0 = (w * p.KT) / 4, kt1 = ((w + 1) * p.KT) / 4;

  // ---- scale | zero table of the tile's columns, first: the entries
  // [n0*G, (n0+BN)*G) of the [N, G] arrays as 16-byte pieces, every load
  // issued before the first LDS write ----
  const int cnt = BN * p.G;
  const int e0 = n0 * p.G;
  const uint32_t sreal = (uint32_t)p.N * (uint32_t)p.G * 2u;
  const int pb = e0 >> 3, pe = (e0 + cnt + 7) >> 3;
  u4 sv[4], zv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int pc = pb + tid + 256 * r;
    const uint32_t off = (uint32_t)pc * 16u;
    const bool ok = pc < pe && off + 16u <= sreal;
    sv[r] = bload16(sr, ok ? off : kOob);
    zv[r] = bload16(zr, ok ? off : kOob);
  }

  // ---- activations: DMA instruction i moves rows 8i..8i+7 of the K-tile;
  // lane l -> row 8i + l/8, LDS position l%8, k-piece (l%8) ^ (row%8) ----
  const int pa = (lane & 7) ^ (lane >> 3);
  const uint32_t rstride = (uint32_t)(8 * p.lda * 2);
  // MFMA A operand of row block i, k-step s: row 16i + c, k-piece 2q + s
  uint32_t ard[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) ard[s] = (uint32_t)(c * 8 + ((2 * q + s) ^ (c & 7)));

  // ---- weights ----
  uint32_t woff[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int col = n0 + 16 * j + c;
    woff[j] = col < p.N ? (uint32_t)(col * p.ldw) + 8u * q : kOob;
  }
  u2v wring[WPF][NB];
  auto load_w = [&](int t, u2v (&dst)[NB]) {
    const bool past = t >= kt1;
    const uint32_t so = past ? 0u : (uint32_t)t * 32u;
    const rsrc_t rr = past ? nullr : wr;
#pragma unroll
    for (int j = 0; j < NB; ++j) dst[j] = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(rr, woff[j], so, 0));
  };

  u4* const slot0 = lds_a0[w];
  u4* const slot1 = lds_a1[w];
  const uint32_t nmask0 = 0x00F0000Fu;
  const uint32_t magic = 0x64006400u;
  const uint32_t sel0 = 0x0c000c00u, sel1 = 0x0c010c01u, sel2 = 0x0c020c02u, sel3 = 0x0c030c03u;
  const uint32_t fm = 0x2C003C00u;   // fp16 pair (1, 1/16)
  const uint32_t fo0 = 0xD480E408u;  // fp16 pair (-1032, -72)

  // Activations: one lane offset (row m0 + l/8, piece pa); row group i adds
  // i*8 rows through the scalar offset.  The buffer's range ends with row
  // M-1 and the range check includes the scalar offset, so rows past M read
  // zeros (they only reach output rows that are never stored).
  const uint32_t adma = (uint32_t)((m0 + (lane >> 3)) * p.lda * 2) + 16u * pa;
  auto dma_one = [&](int t, u4* slot, int i) {
    const bool past = t >= kt1;
    const uint32_t so = past ? 0u : (uint32_t)t * 128u;
    dma16(past ? nullr : ar, slot + 64 * i, adma, so + i * rstride);
  };
  // prologue loads: what the first K-tile's k-step 0 needs (its
  // activations and weights) and the next K-tile's weights; the rest of
  // the pipeline's loads go out when the first K-tile starts (a deep burst
  // issued here would hold back the first data: every CU starts at once)
#pragma unroll
  for (int i = 0; i < 16; ++i) dma_one(kt0, slot0, i);
  load_w(kt0, wring[0]);
  load_w(kt0 + 1, wring[1]);
  // scale | zero table writes (s | z << 16 per entry)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int pc = pb + tid + 256 * r;
    if (pc >= pe) break;
    const uint32_t off = (uint32_t)pc * 16u;
    uint32_t sw[4] = {sv[r].x, sv[r].y, sv[r].z, sv[r].w}, zw[4] = {zv[r].x, zv[r].y, zv[r].z, zv[r].w};
    if (off + 16u > sreal) {   // the piece that straddles the end of the arrays: entry by entry
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t o0 = off + 4u * e, o1 = o0 + 2u;
        sw[e] = bload2(sr, o0 < sreal ? o0 : kOob) | (bload2(sr, o1 < sreal ? o1 : kOob) << 16);
        zw[e] = bload2(zr, o0 < sreal ? o0 : kOob) | (bload2(zr, o1 < sreal ? o1 : kOob) << 16);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int le = pc * 8 + e - e0;
      if (le >= 0 && le < cnt)
        lds_sz[le] = ((sw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) | ((zw[e >> 1] >> (16 * (e & 1))) << 16);
    }
  }
  __syncthreads();
  const uint64_t T1 = __builtin_amdgcn_s_memrealtime();
  uint64_t Tv = 0;
  if (p.trace != nullptr) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); Tv = __builtin_amdgcn_s_memrealtime(); }

  // scale|zero of K-tile t for each block; K-tiles past the wave's range
  // get (0, 0), so their (zero) activations meet zero weights
  auto read_sz = [&](int t, uint32_t (&dst)[NB]) {
    const int g = p.gshift >= 31 ? 0 : min((t * 64 + 16 * q) >> p.gshift, p.G - 1);
    const uint32_t keep = t < kt1 ? 0xFFFFFFFFu : 0u;
#pragma unroll
    for (int j = 0; j < NB; ++j) dst[j] = lds_sz[(16 * j + c) * p.G + g] & keep;
  };

  f4 acc[MBK][NB];
#pragma unroll
  for (int i = 0; i < MBK; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

  uint32_t nmask = nmask0, fo = fo0;
  asm volatile("" : "+v"(nmask), "+v"(fo));

  // One k-step, hand-ordered: region j (weight block j) issues the 8 MFMAs
  // of (af[i], bq[j]) one by one, each followed by a share of the 20 VALU
  // ops that dequantize block j of the next k-step, and by a share of the
  // next k-step's fragment reads and of `extra` (refill loads).
  // early: all of the next k-step's fragments are read at the start (the
  // slot they come from can then be refilled during this k-step)
  auto step = [&](auto earlyc, const h8 (&af)[MBK], const h8 (&bq)[NB], const u4* nsl, int ns, h8 (&naf)[MBK],
                  const u2v (&nwt)[NB], const uint32_t (&nsz)[NB], int nstep, h8 (&nbq)[NB], auto extra) {
    constexpr bool EARLY = decltype(earlyc)::value;
    if (EARLY) {
#pragma unroll
      for (int i = 0; i < MBK; ++i) naf[i] = __builtin_bit_cast(h8, nsl[ard[ns] + 128 * i]);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const uint32_t d = nstep ? nwt[j].y : nwt[j].x;
      const uint32_t e = nsz[j];
      uint32_t x0, x1, x2, x3;
#define MF(i) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc[i][j]) : "v"(bq[j]), "v"(af[i]))
#define PERM(x, sel) asm volatile("v_perm_b32 %0, 0, %1, %2" : "=v"(x) : "v"(d), "s"(sel))
#define ANDOR(x) asm volatile("v_and_or_b32 %0, %0, %1, %2" : "+v"(x) : "v"(nmask), "s"(magic))
#define FMA(x) asm volatile("v_pk_fma_f16 %0, %0, %1, %2" : "+v"(x) : "s"(fm), "v"(fo))
#define MUL(x) asm volatile("v_pk_mul_f16 %0, %1, %0 op_sel_hi:[0,1]" : "+v"(x) : "v"(e))
#define SUB(x) asm volatile("v_pk_add_f16 %0, %0, %1 op_sel:[0,1] neg_lo:[0,1] neg_hi:[0,1]" : "+v"(x) : "v"(e))
#define SB() __builtin_amdgcn_sched_barrier(0)
      // (q-8 exact: nibble pair under 0x6400, then one packed FMA; then
      // RNE(q*s) and RNE(. - z): the reference's two roundings)
      MF(0); PERM(x0, sel0); PERM(x1, sel1); ANDOR(x0); SB();
      MF(1); PERM(x2, sel2); PERM(x3, sel3); ANDOR(x1); SB();
      if (!EARLY && (j * MBK) / NB < ((j + 1) * MBK) / NB)
        naf[(j * MBK) / NB] = __builtin_bit_cast(h8, nsl[ard[ns] + 128 * ((j * MBK) / NB)]);
      SB();
      MF(2); ANDOR(x2); ANDOR(x3); FMA(x0); SB();
      MF(3); FMA(x1); FMA(x2); FMA(x3); SB();
      if (!EARLY && (j * MBK) / NB + 1 < ((j + 1) * MBK) / NB)
        naf[(j * MBK) / NB + 1] = __builtin_bit_cast(h8, nsl[ard[ns] + 128 * ((j * MBK) / NB + 1)]);
      extra(j);
      SB();
      MF(4); MUL(x0); MUL(x1); SUB(x0); SB();
      MF(5); MUL(x2); MUL(x3); SUB(x1); SB();
      MF(6); SUB(x2); SB();
      MF(7); SUB(x3); SB();
      u4 o;
      o.x = x0; o.y = x1; o.z = x2; o.w = x3;
      nbq[j] = __builtin_bit_cast(h8, o);
#undef MF
#undef PERM
#undef ANDOR
#undef FMA
#undef MUL
#undef SUB
#undef SB
    }
  };

  // first k-step's operands (C++ dequant; outside the loop)
  h8 afA[MBK], afB[MBK], bqA[NB], bqB[NB];
  uint32_t sz[NB], sz2[NB];
#pragma unroll
  for (int i = 0; i < MBK; ++i) afA[i] = __builtin_bit_cast(h8, slot0[ard[0] + 128 * i]);
  read_sz(kt0, sz);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const h2 e = as_h2(sz[j]);
    bqA[j] = dq_int4_dword_nat_r(wring[0][j].x, __builtin_shufflevector(e, e, 0, 0),
                                 __builtin_shufflevector(e, e, 1, 1), nmask, magic);
  }

  // K-tile t (t - kt0 = R mod WPF) from slot `cur`; the next K-tile's data is
  // in slot `nxt`.  Weight ring slot R holds K-tile t's weights; it is
  // refilled (K-tile t + WPF) once k-step 0 has dequantized k-step 1.
  auto tile = [&](auto rc, u4* cur, u4* nxt, int t) {
    constexpr int R = decltype(rc)::value;
    constexpr int R1 = (R + 1) % WPF;
    if (R == 0 && t == kt0) {   // the first K-tile: the rest of the prologue
#pragma unroll
      for (int i = 0; i < 16; ++i) dma_one(kt0 + 1, slot1, i);
#pragma unroll
      for (int d = 2; d < WPF; ++d) load_w(kt0 + d, wring[d]);
    }
    read_sz(t + 1, sz2);
    // k-step 0 of tile t: reads all of k-step 1's fragments first; once
    // they are in registers the slot is refilled (K-tile t+2), spread over
    // the rest of the k-step; then the weight slot is refilled
    step(std::true_type{}, afA, bqA, cur, 1, afB, wring[R], sz, 1, bqB, [&](int j) {
      if (j == 0) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if ((i * NB) / 16 == j) dma_one(t + 2, cur, i);
    });
    load_w(t + WPF, wring[R]);
    // k-step 1 of tile t; prepares tile t+1's k-step 0 from slot `nxt`
    step(std::false_type{}, afB, bqB, nxt, 0, afA, wring[R1], sz2, 0, bqA, [&](int) {});
#pragma unroll
    for (int j = 0; j < NB; ++j) sz[j] = sz2[j];
  };
  // WPF K-tiles per iteration (static ring indices: no register copies of
  // loads in flight); a K-tile past the wave's range reads zeros and has
  // zero scales
  static_assert(WPF % 2 == 0, "slot parity");
  int t = kt0;
  uint64_t Tf = 0;
  do {
    tile(std::integral_constant<int, 0>{}, slot0, slot1, t);
    if (t == kt0) Tf = __builtin_amdgcn_s_memrealtime();
    tile(std::integral_constant<int, 1>{}, slot1, slot0, t + 1);
    if (WPF > 2) {
      tile(std::integral_constant<int, 2 % WPF>{}, slot0, slot1, t + 2);
      tile(std::integral_constant<int, 3 % WPF>{}, slot1, slot0, t + 3);
    }
    t += WPF;
  } while (t < kt1);
  const uint64_t T2 = __builtin_amdgcn_s_memrealtime();

  // ---- the four partial tiles meet in LDS ----
  // Block b = i*NB + j is owned by wave b % 4.  Each wave writes its
  // partials of the blocks it does not own into its own activation slots
  // (free once its K loop is done: no barrier before), 1 KiB per block in
  // block order, 16 bytes per lane (conflict-free); after one barrier each
  // owner sums the four partials of its blocks in wave order
  // (deterministic).
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");   // MFMA results retired
#pragma unroll
  for (int i = 0; i < MBK; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) asm volatile("" : "+a"(acc[i][j]));
  // slot of block b in wave ww's region (its blocks not owned by ww, in order)
  auto rslot = [&](int ww, int b) -> f4* {
    const int idx = b - (b > ww ? (b - ww + 3) / 4 : 0);
    return idx < 16 ? (f4*)&lds_a0[ww][0] + idx * 64 : (f4*)&lds_a1[ww][0] + (idx - 16) * 64;
  };
  static_assert(MBK * NB - (MBK * NB) / 4 <= 32, "a wave's partials fit in its two activation slots");
  constexpr int NOWN = (MBK * NB + 3) / 4;
  f4 own[NOWN];
  uint64_t Tb = 0;
  auto gather = [&](auto wc) {
    constexpr int W = decltype(wc)::value;
    // straight from the accumulator registers (no copies through VGPRs);
    // the 24 wait states above cover the MFMA-to-LDS-read dependency
#pragma unroll
    for (int i = 0; i < MBK; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int b = i * NB + j;
        if ((b & 3) != W) {
          const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) f4*)(rslot(W, b) + lane);
          asm volatile("ds_write_b128 %0, %1" :: "v"(la), "a"(acc[i][j]) : "memory");
        }
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();   // every wave's partials are in LDS
    Tb = __builtin_amdgcn_s_memrealtime();
#pragma unroll
    for (int i = 0; i < MBK; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int b = i * NB + j;
        if ((b & 3) != W) continue;
        f4 sum = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {   // wave order: deterministic
          if (ww == W) sum += acc[i][j];
          else sum += rslot(ww, b)[lane];
        }
        own[b >> 2] = sum;
      }
  };
  const uint64_t T3 = __builtin_amdgcn_s_memrealtime();
  if (w == 0) gather(std::integral_constant<int, 0>{});
  else if (w == 1) gather(std::integral_constant<int, 1>{});
  else if (w == 2) gather(std::integral_constant<int, 2>{});
  else gather(std::integral_constant<int, 3>{});
  __syncthreads();   // every partial has been read
  const uint64_t T4 = __builtin_amdgcn_s_memrealtime();
  constexpr int PPR = BN / 8;              // 16-byte pieces per output row
  constexpr int NPC = 128 * PPR / 256;      // pieces per thread
  static_assert(128 * PPR % 256 == 0, "whole pieces per thread");
  const int kind = p.ep.epi;
  if (kind == EPI_NONE && p.vec_store && m0 + 128 <= p.M && n0 + BN <= p.N) {
    // fp16 results staged as [128][SS] halves (rows 16 bytes apart mod 128
    // bytes: the 16 rows of one store group fall in different banks), then
    // 16-byte stores, every LDS read of a thread issued before its stores
    constexpr int SS = BN + 8;
    _Float16* stg = (_Float16*)&lds_a0[0][0];
#pragma unroll
    for (int u = 0; u < NOWN; ++u) {
      const int b = 4 * u + w;
      if (b >= MBK * NB) break;
      const int i = b / NB, j = b - i * NB;
      typedef _Float16 h4 __attribute__((ext_vector_type(4)));
      *(h4*)&stg[(16 * i + c) * SS + 16 * j + 4 * q] =
          (h4){(_Float16)own[u][0], (_Float16)own[u][1], (_Float16)own[u][2], (_Float16)own[u][3]};
    }
    __syncthreads();
    const uint64_t T5 = __builtin_amdgcn_s_memrealtime();
    h8 pv[NPC];
#pragma unroll
    for (int e = 0; e < NPC; ++e) {
      const int pc = tid + 256 * e;
      const int r = pc / PPR, cc = 8 * (pc - r * PPR);
      pv[e] = *(const h8*)&stg[r * SS + cc];
    }
#pragma unroll
    for (int e = 0; e < NPC; ++e) {
      const int pc = tid + 256 * e;
      const int r = pc / PPR, cc = 8 * (pc - r * PPR);
      *(h8*)(p.C + (int64_t)(m0 + r) * p.ldc + n0 + cc) = pv[e];
    }
    if (p.trace != nullptr && lane == 0) {
      uint64_t* o = p.trace + ((size_t)blockIdx.x * 4 + w) * 8;
      o[5] = T5;
    }
  } else {
    // fp32 sums staged as [128][RS]; the epilogue is applied per element,
    // then fp16 rounding and 16-byte stores where the rows allow
    constexpr int RS = BN + 4;
    float* res = (float*)&lds_a0[0][0];
    static_assert(128 * RS * 4 <= 4 * 1024 * 16, "result tile fits the first activation array");
    // owned block b = 4u + w: row 16i + c, columns 16j + 4q .. +3
#pragma unroll
    for (int u = 0; u < NOWN; ++u) {
      const int b = 4 * u + w;
      if (b >= MBK * NB) break;
      const int i = b / NB, j = b - i * NB;
      *(f4*)&res[(16 * i + c) * RS + 16 * j + 4 * q] = own[u];
    }
    __syncthreads();
    for (int pc = tid; pc < 128 * PPR; pc += 256) {
      const int r = pc / PPR, cc = 8 * (pc - r * PPR);
      const int row = m0 + r, col = n0 + cc;
      if (row >= p.M || col >= p.N) continue;
      const f4 v0 = *(const f4*)&res[r * RS + cc], v1 = *(const f4*)&res[r * RS + cc + 4];
      float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      const int ncol = min(8, p.N - col);
      if (kind != EPI_NONE) {
        for (int e = 0; e < ncol; ++e) v[e] = epi_apply(v[e], (int64_t)row, col + e, p.ep);
      }
      _Float16* dst = p.C + (int64_t)row * p.ldc + col;
      if (p.vec_store && ncol == 8) {
        h8 hv;
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[e] = (_Float16)v[e];
        *(h8*)dst = hv;
      } else {
        for (int e = 0; e < ncol; ++e) dst[e] = (_Float16)v[e];
      }
    }
  }
  if (p.trace != nullptr && lane == 0) {
    uint64_t* o = p.trace + ((size_t)blockIdx.x * 4 + w) * 8;
    o[0] = T0; o[1] = T1; o[2] = T2; o[4] = T4; o[6] = __builtin_amdgcn_s_memrealtime(); o[7] = Tf; o[3] = Tv;
  }
}

constexpr int kNB = 5;

bool shape_ok(const LinearArgs& a) {
  if (a.fmt != FMT_INT4 || a.epi == EPI_SWIGLU || a.prenorm) return false;
  if (a.M < 1 || a.N < 1 || a.K < 64 || a.K % 64 != 0) return false;
  if (a.lda % 8 != 0 || ((uintptr_t)a.A & 15) != 0) return false;           // 16-byte activation pieces
  if (a.ldw % 8 != 0 || ((uintptr_t)a.W & 7) != 0) return false;            // 8-byte weight loads
  const bool per_channel = a.g >= a.K;
  if (!per_channel && (a.g < 16 || (a.g & (a.g - 1)) != 0)) return false;  // a lane's 16 k in one group
  // 32-bit buffer offsets
  if ((int64_t)a.M * a.lda * 2 >= (1ll << 31) || (int64_t)a.N * a.ldw >= (1ll << 31)) return false;
  if ((int64_t)a.N * a.G * 2 >= (1ll << 31)) return false;
  if ((int64_t)16 * kNB * a.G > G16_SZT) return false;
  return a.zeros != nullptr;
}

}  // namespace

bool gemm16_supported(const LinearArgs& a) { return shape_ok(a); }

int gemm16_workgroups(const LinearArgs& a) {
  return ((a.M + 127) / 128) * ((a.N + 16 * kNB - 1) / (16 * kNB));
}

hipError_t gemm16_launch(const LinearArgs& a, hipStream_t s, uint64_t* trace) {
  if (!shape_ok(a)) return hipErrorInvalidValue;
  G16Args k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.ep = a.epi_args();
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.G = a.G;
  k.gshift = a.g >= a.K ? 31 : __builtin_ctz((unsigned)a.g);
  k.nbm = (a.M + 127) / 128;
  k.KT = a.K / G16_KT;
  const int nwg = gemm16_workgroups(a);
  k.xcd = nwg % 8 == 0;
  k.vec_store = (a.ldc % 8 == 0) && (((uintptr_t)a.C & 15) == 0);
  // bytes of A up to the end of its last row, of W, of one scale array
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  k.w_bytes = (uint32_t)((int64_t)(a.N - 1) * a.ldw + a.K / 2);
  k.s_bytes = (uint32_t)((int64_t)a.N * a.G * 2);
  k.trace = trace;
  hipLaunchKernelGGL((gemm16_kernel<kNB>), dim3(nwg), dim3(256), 0, s, k);
  return hipGetLastError();
}

}  // namespace mq
