// Prefill dequant GEMM (M >= 17): C = epi(A . deq(W)^T), fp16 products
// accumulated in fp32 by v_mfma_f32_32x32x16_f16, one rounding to fp16.
//
// Replaces dequant_matmul_int4_fp16 / dequant_matmul_int8_fp16
// (shaders/matmul_dequant_kernel.metal:55-223, :351-479; dispatched at
// src/ops/matmul.mm:1011-1021).
//
// Shaped by measurements on gfx950 (per CU: 4 SIMDs, one texture unit):
//   * a v_mfma_f32_32x32x16_f16 stream reaches ~2.15 PFLOP/s on the chip, and
//     up to 8 independent VALU instructions per MFMA issue in its shadow;
//   * one 1 KiB ds_read_b128 per MFMA (per wave) halves the MFMA rate (LDS
//     delivers ~128 B/clk per CU);
//   * the texture unit serves ~64 B/clk per CU when four adjacent lanes read
//     64 contiguous bytes, but only ~16 B/clk when every lane reads its own
//     row (the MFMA operand layout: 32 rows per load instruction).
//
//  * Workgroup = 4 waves (one per SIMD) on one output tile of BM = 32*MB rows
//    by BN (<= 32*NB) columns; wave w takes the w-th quarter of the K-tiles
//    (64 k each).  Every weight is loaded and dequantized once per
//    workgroup, every activation moved once per workgroup.
//  * Activations: direct-to-LDS loads (buffer_load ... lds), fully
//    coalesced, into a per-wave double buffer, XOR-swizzled so that the MFMA
//    fragment reads (one row per lane) are bank-conflict free.
//  * Weights: loaded straight into B operands (lane r + 32h holds k
//    32h..32h+31 of column r, 16 bytes) and dequantized in registers with
//    the exact two-rounding formula; scales and zeros come from a table of
//    the workgroup's rows filled once with coalesced loads.
//  * MB = 4 A blocks per weight block keep the dequant at ~5 VALU per MFMA.
//    The MFMAs of k-step s are interleaved (scheduling groups) with the
//    dequant of step s+1 and the refill loads of later K-tiles: one wave per
//    SIMD issues in order, so MFMA and VALU overlap only when interleaved.
//  * After the K loop the four partial tiles meet in LDS: each wave owns a
//    quarter of the 32x32 blocks (SwiGLU: gate/up block pairs), receives the
//    other waves' partials of those blocks and sums the four in wave order
//    (deterministic), applies the epilogue and stores fp16.
//  * Tile widths are chosen per shape so that the tiles cover the CUs once
//    (e.g. 128 x 80 for the Llama-3.2-3B QKV shape: 4 x 64 = 256 tiles);
//    blocks past the tile width are masked (their loads read nothing).
//  * Workgroups of one XCD take a contiguous run of tiles, M-block fastest, so
//    the workgroups that share a weight slice share an L2.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <algorithm>
#include <cmath>

namespace mq {
namespace {

constexpr int KTK = 64;    // k per K-tile
constexpr int NWV = 4;     // waves per workgroup, each a quarter of the K-tiles
// K-tiles of weights in flight ahead of the dequant.  A tile issues 16 + 3
// vector loads (MB = 4, NB = 3); two tiles of activations and three of
// weights keep at most 41 loads outstanding, under the 63 the load counter
// can track.
constexpr int WPF = 2;
constexpr int WSL = WPF + 1;   // weight slots
constexpr int ASLOT = 1024;    // 16-byte pieces per wave per activation slot (128 rows x 128 bytes)
constexpr int SZT = 8192;      // scale (and zero) entries of the workgroup's rows (16 KiB each)
constexpr int kBlockF = 64 * 16;   // floats of one 32x32 fp32 block, lane-major

struct GemmWArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros;
  EpiArgs ep;
  _Float16* C; int64_t ldc;
  int M, N, K, G, F, gshift;
  int BN;            // output columns per tile (SwiGLU: gate columns)
  int nbm, nbn, xcd_remap;
  int KT;            // K-tiles
  int KP, tiles;     // K parts (workgroups per tile) and output tiles
  float* part;       // K > 1 parts: [KP][tiles][MB*NB blocks][1024] fp32 partial sums
  uint32_t* cnt;     // K > 1 parts: per-tile arrival counts, zero between launches
  uint32_t a_bytes, w_bytes, s_bytes, z_bytes;
};

template <int FMT>
struct WTile {            // one K-tile of one weight column for this lane half
  u4 v[FMT == FMT_INT4 ? 1 : 2];
};

__device__ __forceinline__ void lds_dma16(rsrc_t r, u4* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// KS: K split over p.KP workgroups per tile (a separate instantiation, so
// that the one-part kernel's code is not shaped by the split's epilogue)
template <int FMT, bool SWI, int MB, int NB, bool KS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemmw_kernel(GemmWArgs p) {
  // Activation slots (separate arrays, so that the compiler's load-counter
  // waits tell a slot's DMA from the other's) and the scale tables; after
  // the K loop the same 160 KiB hold the partial tiles of the reduction.
  __shared__ u4 lds_a0[NWV][ASLOT];
  __shared__ u4 lds_a1[NWV][ASLOT];
  __shared__ _Float16 lds_s[SZT];
  __shared__ _Float16 lds_z[SZT];
  constexpr int WB = FMT == FMT_INT4 ? 32 : 64;   // weight bytes per column per K-tile
  static_assert(!SWI || NB % 2 == 0, "SwiGLU pairs gate and up blocks");
  static_assert(MB * NB * 3 * kBlockF * 4 <= 2 * NWV * ASLOT * 16 + 2 * SZT * 2, "reduction buffer");

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;

  int id = blockIdx.x;
  if (p.xcd_remap) {   // workgroup i runs on XCD i % 8: give each XCD a contiguous run of tiles
    const int per = gridDim.x >> 3;
    id = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  }
  // K part major: the workgroups of one XCD share a K range of the activations
  const int kp = KS ? id / p.tiles : 0;
  const int otile = KS ? id - kp * p.tiles : id;   // output tile
  const int nb = otile / p.nbm, mb = otile - nb * p.nbm;
  const int m0 = mb * 32 * MB;
  const int n0 = nb * p.BN;

  const rsrc_t ar = make_rsrc(p.A, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  const rsrc_t sr = make_rsrc(p.scales, p.s_bytes);
  const rsrc_t zr = make_rsrc(p.zeros, p.z_bytes);

  // ---- this wave's K-tiles ----
  const int kb = KS ? (kp * p.KT) / p.KP : 0, ke = KS ? ((kp + 1) * p.KT) / p.KP : p.KT;   // this K part
  const int kt0 = kb + (w * (ke - kb)) / NWV, kt1 = kb + ((w + 1) * (ke - kb)) / NWV;

  // ---- activations: DMA into LDS, fully coalesced ----
  // Load instruction i moves rows 8i..8i+7 of the tile: lane l takes row
  // 8i + l/8 and stores at 16-byte slot l%8 of that row's 128 bytes; the
  // slot holds k-piece (l%8) ^ (row % 8), so that the MFMA reads below (32
  // rows, one piece each) fall in different banks.
  const int pa = (lane & 7) ^ (lane >> 3);          // k-piece this lane moves
  uint32_t adma[MB * 4];
#pragma unroll
  for (int i = 0; i < MB * 4; ++i) {
    const int row = m0 + 8 * i + (lane >> 3);
    adma[i] = row < p.M ? (uint32_t)(row * p.lda * 2) + 16u * pa : kOob;
  }
  // the last K-tile may end past K (K % 64 == 32): its pieces past K read nothing
  const bool apast = (p.KT - 1) * KTK + 8 * pa >= p.K;
  // (tiles past the wave's range move nothing: out-of-range offsets)
  auto dma_a = [&](int t, u4* slot) {
    const bool past = t >= kt1;
    const uint32_t so = past ? 0u : (uint32_t)t * (KTK * 2);
    const bool cut = past || (t == p.KT - 1 && apast);
#pragma unroll
    for (int i = 0; i < MB * 4; ++i) lds_dma16(ar, slot + 64 * i, cut ? kOob : adma[i], so);
  };
  // MFMA A operand of block i, step s: row 32i + r, k 32h + 8s..+7 = piece 4h + s
  uint32_t ard[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) ard[s] = (uint32_t)(r * 8 + ((4 * h + s) ^ (r & 7)));

  // ---- weights: straight into B operands ----
  uint32_t woff[NB];
  int wrow_of[NB];
  bool wok[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    int c, wrow, lim;
    if (SWI) {
      c = 32 * (j >> 1) + r;
      wrow = (j & 1) ? p.F + n0 + c : n0 + c;
      lim = p.F;
    } else {
      c = 32 * j + r;
      wrow = n0 + c;
      lim = p.N;
    }
    wok[j] = c < p.BN && n0 + c < lim;
    wrow_of[j] = wrow;
    woff[j] = wok[j] ? (uint32_t)(wrow * p.ldw) + (uint32_t)(WB / 2) * h : kOob;
  }
  const bool wpast = (p.KT - 1) * KTK + 32 * h >= p.K;

  // scale/zero table: the workgroup's weight rows x all groups, the layout
  // of the [N, G] arrays (SwiGLU: the gate rows, then the up rows at row BN)
  auto lrow = [&](int j) { return SWI ? ((j & 1) ? p.BN : 0) + 32 * (j >> 1) + r : 32 * j + r; };

  WTile<FMT> wreg[WSL][NB];
  auto load_w = [&](int t, WTile<FMT> (&dst)[NB]) {
    const bool past = t >= kt1;
    const uint32_t so = past ? 0u : (uint32_t)t * WB;
    const bool cut = past || (t == p.KT - 1 && wpast);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const uint32_t vo = cut ? kOob : woff[j];
#pragma unroll
      for (int e = 0; e < (FMT == FMT_INT4 ? 1 : 2); ++e)
        dst[j].v[e] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wr, vo + 16 * e, so, 0));
    }
  };
  // scale|zero of tile t for each block (tiles past the range read entry 0;
  // a last K-tile half past K keeps the row's last group, not the next row's)
  auto read_sz = [&](int t, uint32_t (&dst)[NB]) {
    const int tc = t < kt1 ? t : kt0;
    const int g = p.gshift >= 31 ? 0 : min((tc * KTK + 32 * h) >> p.gshift, p.G - 1);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int e = lrow(j) * p.G + g;
      dst[j] = (uint32_t)__builtin_bit_cast(uint16_t, lds_s[e]) | ((uint32_t)__builtin_bit_cast(uint16_t, lds_z[e]) << 16);
    }
  };

  // nibble mask in a VGPR, the fp16 1024 pair in an SGPR (one v_and_or_b32 per pair)
  uint32_t nmask = 0x00F0000Fu;
  asm volatile("" : "+v"(nmask));
  const uint32_t magic = 0x64006400u;

  // dequantized B operands of one k-step, all blocks
  auto dequant = [&](const WTile<FMT> (&wt)[NB], const uint32_t (&sz)[NB], int s, h8 (&bq)[NB]) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      // broadcast halves: the packed ops' operand selectors read them in place
      const h2 e = as_h2(sz[j]);
      const h2 s2 = __builtin_shufflevector(e, e, 0, 0);
      const h2 z2 = __builtin_shufflevector(e, e, 1, 1);
      if (FMT == FMT_INT4) {
        const u4 v = wt[j].v[0];
        const uint32_t d = s == 0 ? v.x : s == 1 ? v.y : s == 2 ? v.z : v.w;
        bq[j] = dq_int4_dword_nat_r(d, s2, z2, nmask, magic);
      } else {
        const u4 v = wt[j].v[s >> 1];
        const uint32_t d0 = (s & 1) ? v.z : v.x, d1 = (s & 1) ? v.w : v.y;
        h2 q0, q1, q2, q3;
        dq_int8_dword(d0, s2, z2, q0, q1);
        dq_int8_dword(d1, s2, z2, q2, q3);
        h8 b;
        b.s01 = q0; b.s23 = q1; b.s45 = q2; b.s67 = q3;
        bq[j] = b;
      }
    }
  };

  f16v acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = (f16v){};

  // ---- pipeline ----
  // Tile t (counted from the wave's first): activations in LDS slot t & 1,
  // weights in wreg[t % 3], scales in szr[t & 1].  Step s of tile t issues
  // its MFMAs with bq[s & 1] and the A fragments of step s while the weights
  // of step s+1 (or step 0 of tile t+1) are dequantized and the A fragments
  // of step s+1 are read.  After the tile its slots are refilled: activations
  // of tile t+2, weights of tile t+3.
  u4* const slot0 = lds_a0[w];
  u4* const slot1 = lds_a1[w];
  dma_a(kt0, slot0);
#pragma unroll
  for (int d = 0; d < WPF; ++d) load_w(kt0 + d, wreg[d]);
  dma_a(kt0 + 1, slot1);
  load_w(kt0 + WPF, wreg[WPF]);
  // ---- scale / zero table, filled by the whole workgroup with 16-byte
  // loads of the contiguous row ranges (after the first tiles' loads: one
  // memory round trip covers both) ----
  {
    const int nr0 = max(0, min(p.BN, (SWI ? p.F : p.N) - n0));
    const int cnt = nr0 * p.G;                       // entries per range
    const int nrange = SWI ? 2 : 1;
    const uint32_t real = (uint32_t)p.N * (uint32_t)p.G * 2u;   // bytes of the scale array
    for (int q = 0; q < nrange; ++q) {
      const int e0 = (q ? p.F + n0 : n0) * p.G;      // first entry of the range
      const int d0 = q ? p.BN * p.G : 0;             // its place in the table
      const int pb = e0 >> 3, pe = (e0 + cnt + 7) >> 3;
      for (int pc = pb + tid; pc < pe; pc += 64 * NWV) {
        const uint32_t off = (uint32_t)pc * 16u;
        uint32_t sw[4], zw[4];
        if (off + 16u <= real) {
          const u4 sv = bload16(sr, off), zv = bload16(zr, off);
          sw[0] = sv.x; sw[1] = sv.y; sw[2] = sv.z; sw[3] = sv.w;
          zw[0] = zv.x; zw[1] = zv.y; zw[2] = zv.z; zw[3] = zv.w;
        } else {   // the piece that straddles the end of the arrays: entry by entry
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t o0 = off + 4u * e, o1 = o0 + 2u;
            sw[e] = bload2(sr, o0 < real ? o0 : kOob) | (bload2(sr, o1 < real ? o1 : kOob) << 16);
            zw[e] = bload2(zr, o0 < real ? o0 : kOob) | (bload2(zr, o1 < real ? o1 : kOob) << 16);
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int le = pc * 8 + e - e0;
          if (le >= 0 && le < cnt) {
            lds_s[d0 + le] = __builtin_bit_cast(_Float16, (uint16_t)(sw[e >> 1] >> (16 * (e & 1))));
            lds_z[d0 + le] = __builtin_bit_cast(_Float16, (uint16_t)(zw[e >> 1] >> (16 * (e & 1))));
          }
        }
      }
    }
    __syncthreads();
  }
  uint32_t szr[2][NB];
  read_sz(kt0, szr[0]);
  h8 bq[2][NB];
  dequant(wreg[0], szr[0], 0, bq[0]);

  auto tile = [&](auto tc, int t) {
    constexpr int T = decltype(tc)::value;   // t % 6
    constexpr int AS = T & 1, WS = T % WSL, WN = (T + 1) % WSL;
    const u4* sl = AS ? slot1 : slot0;
    // all A fragments of the tile at once: the slot is then free for the
    // refill, which can be spread over the rest of the tile
    h8 af[4][MB];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < MB; ++i) af[s][i] = __builtin_bit_cast(h8, sl[ard[s] + 256 * i]);
    read_sz(t + 1, szr[AS ^ 1]);
    auto step = [&](int s) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s][i], bq[s & 1][j], acc[i][j], 0, 0, 0);
      if (s < 3) dequant(wreg[WS], szr[AS], s + 1, bq[(s + 1) & 1]);
      else dequant(wreg[WN], szr[AS ^ 1], 0, bq[0]);
    };
    // One wave per SIMD issues in order: each MFMA is interleaved with the
    // dequant VALU work (and later with the refill loads), so that they run
    // in the MFMA's shadow.
    step(0);
#pragma unroll
    for (int m = 0; m < MB * NB; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // up to six VALU
    }
    // the slot's reads (and the scale reads) have completed before the DMA
    // overwrites it
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    step(1);
    step(2);
    step(3);
    dma_a(t + 2, AS ? slot1 : slot0);
    load_w(t + WSL, wreg[WS]);
    constexpr int NVM = MB * 4 + NB * (FMT == FMT_INT4 ? 1 : 2);   // refill loads
#pragma unroll
    for (int m = 0; m < 3 * MB * NB; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
      if (m % 2 == 0 && m / 2 < NVM) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // one refill load
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // up to six VALU
    }
    // keep the refills in this tile: the scheduler would otherwise sink them
    // to their uses a tile or two later, next to a wait for them
    __builtin_amdgcn_sched_barrier(0);
  };
  int t = kt0;
  for (; t + 6 <= kt1; t += 6) {
    tile(std::integral_constant<int, 0>{}, t);
    tile(std::integral_constant<int, 1>{}, t + 1);
    tile(std::integral_constant<int, 2>{}, t + 2);
    tile(std::integral_constant<int, 3>{}, t + 3);
    tile(std::integral_constant<int, 4>{}, t + 4);
    tile(std::integral_constant<int, 5>{}, t + 5);
  }
  // remaining 0..5 tiles (uniform branches)
  if (t < kt1) tile(std::integral_constant<int, 0>{}, t);
  if (t + 1 < kt1) tile(std::integral_constant<int, 1>{}, t + 1);
  if (t + 2 < kt1) tile(std::integral_constant<int, 2>{}, t + 2);
  if (t + 3 < kt1) tile(std::integral_constant<int, 3>{}, t + 3);
  if (t + 4 < kt1) tile(std::integral_constant<int, 4>{}, t + 4);

  // ---- the four partial tiles meet in LDS ----
  // (accumulators stay in place: the fence names them as AGPR operands)
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(acc[i][j]));
  // every wave is done with its activation slots and the scale table
  __syncthreads();
  // Unit u (block (i, j), or the gate/up block pair (i, 2q..2q+1) for
  // SwiGLU) is owned by wave u % 4.  The three other waves write their
  // partials of its blocks to slot (block, rank), rank = writer index among
  // the non-owners, 4 KiB each: slots 0..15 in the first activation array,
  // 16..31 in the second, 32..35 in the scale table, 36..39 in the zero
  // table.  Within a slot, quad q of the 16 accumulator values of lane l
  // sits at 16 bytes * (64 q + l) (conflict-free 16-byte LDS accesses).
  // The code is specialised per wave, so every block index is a constant.
  auto red_slot = [&](int k) -> float* {
    if (k < 16) return (float*)&lds_a0[0][0] + k * kBlockF;
    if (k < 32) return (float*)&lds_a1[0][0] + (k - 16) * kBlockF;
    return (float*)(k < 36 ? (void*)&lds_s[0] : (void*)&lds_z[0]) + ((k - 32) & 3) * kBlockF;
  };
  constexpr int NBLK = SWI ? 2 : 1;          // blocks per unit
  constexpr int NU = MB * NB / NBLK;         // units
  const int rbase = m0 + 4 * h;
  // epilogue and fp16 stores of unit (i, jq) from its fp32 sums
  auto emit = [&](int i, int jq, const f16v (&sum)[SWI ? 2 : 1]) {
    // lane holds D[row = 8*(v/4) + 4*h + v%4][col = r] of the block; the
    // rows are checked against M only in the last M block, and the
    // epilogue kind is switched on once per block
    const int c = 32 * jq + r;
    const int col = n0 + c;
    const int row0 = rbase + 32 * i;
    if (c >= p.BN || col >= (SWI ? p.F : p.N)) return;
    _Float16* cp = p.C + (int64_t)row0 * p.ldc + col;
    float outv[16];
    if (SWI) {
#pragma unroll
      for (int v = 0; v < 16; ++v) outv[v] = silu_f32((float)(_Float16)sum[0][v]) * (float)(_Float16)sum[NBLK - 1][v];
    } else {
      const int kind = p.ep.epi;
      const float bv = epi_needs_bias(kind) ? (float)((const _Float16*)p.ep.bias)[col] : 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) outv[v] = sum[0][v] + bv;
      if (kind == EPI_RESIDUAL) {
        const _Float16* rp = (const _Float16*)p.ep.resid + (int64_t)row0 * p.ep.ldr + col;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int dr = 8 * (v >> 2) + (v & 3);
          if (row0 + dr < p.M) outv[v] += (float)rp[(int64_t)dr * p.ep.ldr];
        }
      } else if (kind == EPI_BIAS_SILU) {
#pragma unroll
        for (int v = 0; v < 16; ++v) outv[v] = silu_f32(outv[v]);
      } else if (kind == EPI_BIAS_RELU) {
#pragma unroll
        for (int v = 0; v < 16; ++v) outv[v] = fmaxf(outv[v], 0.0f);
      }
    }
    if (m0 + 32 * (i + 1) <= p.M) {
#pragma unroll
      for (int v = 0; v < 16; ++v) cp[(int64_t)(8 * (v >> 2) + (v & 3)) * p.ldc] = (_Float16)outv[v];
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int dr = 8 * (v >> 2) + (v & 3);
        if (row0 + dr < p.M) cp[(int64_t)dr * p.ldc] = (_Float16)outv[v];
      }
    }
  };
  // partial sums of K part q, block blk of this tile: 16 values per lane,
  // value v of lane l at float 64 v + l (coalesced)
  auto part_of = [&](int q, int blk) -> float* {
    return p.part + (((int64_t)q * p.tiles + otile) * (MB * NB) + blk) * kBlockF + lane;
  };
  auto finish = [&](auto wc) {
    constexpr int W = decltype(wc)::value;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int own = (SWI ? i * (NB / 2) + (j >> 1) : i * NB + j) & 3;
        if (own != W) {
          float* dst = red_slot((i * NB + j) * 3 + (W < own ? W : W - 1)) + lane * 4;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *(f4*)(dst + q * 256) = (f4){acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
      }
    __syncthreads();
#pragma unroll
    for (int u = W; u < NU; u += 4) {
      const int i = u / (NB / NBLK), jq = u - i * (NB / NBLK);
      f16v sum[NBLK];
#pragma unroll
      for (int b = 0; b < NBLK; ++b) {
        const int jj = NBLK * jq + b;
        sum[b] = (f16v){};
#pragma unroll
        for (int ww = 0; ww < NWV; ++ww) {   // wave order: deterministic
          if (ww == W) {
            sum[b] += acc[i][jj];
          } else {
            const float* src = red_slot((i * NB + jj) * 3 + (ww < W ? ww : ww - 1)) + lane * 4;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f4 v = *(const f4*)(src + q * 256);
              sum[b][4 * q] += v[0]; sum[b][4 * q + 1] += v[1]; sum[b][4 * q + 2] += v[2]; sum[b][4 * q + 3] += v[3];
            }
          }
        }
      }
      if constexpr (!KS) {
        emit(i, jq, sum);
      } else {   // this K part's sums
#pragma unroll
        for (int b = 0; b < NBLK; ++b) {
          float* dst = part_of(kp, i * NB + NBLK * jq + b);
#pragma unroll
          for (int v = 0; v < 16; ++v)
            __hip_atomic_store(dst + 64 * v, sum[b][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
      }
    }
    if constexpr (!KS) return;
    // Split K: the last of the tile's K parts to arrive sums all parts in
    // part order (deterministic) and stores; no workgroup waits for another.
    // Ordering: every access to the partials is a system-scope atomic
    // (stores written through to memory, loads served from memory); each
    // wave waits for its stores to be acknowledged before the barrier that
    // precedes the count, so the count is taken only after every partial of
    // this part is in memory.  That is the gfx950 lowering of a system-scope
    // release (and, on the reading side, acquire) without the L2 writeback
    // and invalidate, which exist to publish non-atomic accesses (none are
    // made here) and measured 2-3x slower for this kernel as a whole.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();   // also: every wave is done with the reduction slots
    uint32_t* flag = (uint32_t*)&lds_s[0];
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(p.cnt + otile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      *flag = prev == (uint32_t)(p.KP - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (*flag == 0u) return;
#pragma unroll
    for (int u = W; u < NU; u += 4) {
      const int i = u / (NB / NBLK), jq = u - i * (NB / NBLK);
      f16v sum[NBLK];
#pragma unroll
      for (int b = 0; b < NBLK; ++b) {
        sum[b] = (f16v){};
        for (int q = 0; q < p.KP; ++q) {
          const float* src = part_of(q, i * NB + NBLK * jq + b);
#pragma unroll
          for (int v = 0; v < 16; ++v)
            sum[b][v] += __hip_atomic_load(src + 64 * v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
      }
      emit(i, jq, sum);
    }
    if (tid == 0) __hip_atomic_store(p.cnt + otile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);   // for the next launch
  };
  switch (w) {
    case 0: finish(std::integral_constant<int, 0>{}); break;
    case 1: finish(std::integral_constant<int, 1>{}); break;
    case 2: finish(std::integral_constant<int, 2>{}); break;
    default: finish(std::integral_constant<int, 3>{}); break;
  }
}

// ---- host side: tile planning and launch ----

struct WPlan {
  int MB, NB, BN, nbm, nbn, KP;
  size_t ws_bytes;
  bool ok;
};

constexpr size_t kCntBytesW = 65536;   // per-tile counters at the start of the workspace

int gshift_of(const LinearArgs& a) {
  if (a.G == 1) return 31;
  for (int b = 5; b < 31; ++b)
    if (a.g == (1 << b)) return b;
  return -1;
}

// The scale table holds the workgroup's weight rows x all groups.
bool sz_table_fits(const LinearArgs& a, int BN) {
  return (int64_t)(a.epi == EPI_SWIGLU ? 2 * BN : BN) * a.G <= SZT;
}

// Time model of one tile (microseconds at ~2.1 GHz): MFMA issue, dequant
// VALU, texture-unit requests and the tile's weight bytes at its share of
// ~6 TB/s; the launch takes ceil(tiles / CUs) tile times (one workgroup per
// CU).
WPlan plan(const LinearArgs& a, int cus, bool allow_split) {
  WPlan best{};
  best.ok = false;
  double best_t = 1e300;
  const int swi = a.epi == EPI_SWIGLU;
  const int ncols = swi ? a.F : a.N;
  const double kt = std::ceil(a.K / 64.0);
  const double bpw = a.fmt == FMT_INT4 ? 0.5 : 1.0;
  // 4 A blocks per weight block keep the dequant VALU in the MFMA shadow;
  // fewer only for few rows (one block of 32 rows: M <= 32, measured 17 %
  // faster than two at M = 32, K = 3584, N = 14336)
  const int mbs[3] = {4, 2, 1};
  for (int MB : mbs) {
    if ((MB == 2 && a.M > 96) || (MB == 1 && a.M > 32)) continue;
    for (int NB = 2; NB <= 6; ++NB) {
      if (swi && NB % 2) continue;
      // the instantiated shapes (launch3); MB * NB <= 12 accumulator blocks
      const bool inst = MB == 4 ? (NB == 2 || (NB == 3 && !swi))
                                : MB == 2 ? (NB == 2 || NB == 4 || NB == 6 || (NB == 3 && !swi)) : NB == 2;
      if (!inst) continue;
      const int maxbn = swi ? 16 * NB : 32 * NB;
      for (int BN = maxbn - 16; BN <= maxbn; BN += 16) {
        if (BN <= 0 || !sz_table_fits(a, BN)) continue;
        const int nbm = (a.M + 32 * MB - 1) / (32 * MB);
        const int nbn = (ncols + BN - 1) / BN;
        const int64_t tiles = (int64_t)nbm * nbn;
        if (tiles > 0x7fffffff / 64) continue;
        const double per = kt / 4.0;   // K-tiles per wave
        const double t_mfma = MB * NB * per * 4 * 32 / 2100.0;
        const double t_valu = NB * per * 4 * (a.fmt == FMT_INT4 ? 21 : 19) * 4 / 2100.0;
        // the CU's texture unit: 64-byte requests, one per clock; the
        // activation DMA takes 16 per 1 KiB, a weight load 64 (one row per lane)
        const double t_ta = per * NWV * (MB * 4 * 16 + NB * 64 * (a.fmt == FMT_INT4 ? 1 : 2)) / 2100.0;
        const double wbytes = (double)(swi ? 2 * BN : BN) * a.K * bpw;
        const double active = (double)std::min<int64_t>(tiles, cus);
        const double t_mem = wbytes / (6.0e6 / active);
        const double t = std::ceil((double)tiles / cus) * std::max(std::max(t_mfma, t_ta), std::max(t_valu, t_mem));
        if (t < best_t * 0.999) {
          best_t = t;
          best = WPlan{MB, NB, BN, nbm, nbn, 1, 0, true};
        }
      }
    }
  }
  // K split over workgroups, where the tiles above leave at least half the
  // CUs idle: candidates of 2 weight blocks (wider tiles measured slower at
  // these shapes) and 1, 2 or 4 A blocks, with 1..8 K parts of at least 8 K-tiles each, priced by a
  // launch-time model fitted to 290 measured launches (int4, M = 17..128, K
  // = 2048..18944): per-wave K-tiles times the tile's MFMA, dequant and
  // activation work, rounds of workgroups over the CUs, and for K parts a
  // fixed cost plus the last arriver's reads of the parts.
  if (best.ok && allow_split && (int64_t)best.nbm * best.nbn * 2 <= cus) {
    auto fitted = [&](int MB, int NB, int64_t tiles, int KP) {
      const double per = kt / KP / 4.0;
      const double rounds = std::ceil((double)(tiles * KP) / cus);
      const double rp = rounds * per;
      const double sp = KP > 1 ? 1.0 : 0.0;
      return -5.09 + rp * (0.1544 + 0.1768 * MB * NB + 0.0858 * NB - 0.1602 * MB) + sp * (2.78 + 0.1575 * KP * MB * NB) +
             11.39 * rounds;
    };
    double fbest = fitted(best.MB, best.NB, (int64_t)best.nbm * best.nbn, 1);
    const int NB = 2;
    // one A block per tile where M <= 32 (12-17 % faster than two at M = 16..32)
    for (int MB : mbs) {
      if ((MB == 2 && a.M > 96) || (MB == 1 && a.M > 32)) continue;
      for (int BN = (swi ? 16 : 32) * NB - 16; BN <= (swi ? 16 : 32) * NB; BN += 16) {
        if (BN <= 0 || !sz_table_fits(a, BN)) continue;
        const int nbm = (a.M + 32 * MB - 1) / (32 * MB);
        const int nbn = (ncols + BN - 1) / BN;
        const int64_t tiles = (int64_t)nbm * nbn;
        if (tiles * 4 > (int64_t)kCntBytesW) continue;
        for (int KP = 2; KP <= 8 && tiles * KP <= cus && kt >= 8.0 * KP; ++KP) {
          const double f = fitted(MB, NB, tiles, KP);
          if (f < fbest * 0.999) {
            fbest = f;
            best = WPlan{MB, NB, BN, nbm, nbn, KP, 0, true};
          }
        }
      }
    }
  }
  if (best.ok && best.KP > 1)
    best.ws_bytes = kCntBytesW + (size_t)best.KP * best.nbm * best.nbn * best.MB * best.NB * kBlockF * 4;
  return best;
}

template <int FMT, bool SWI, int MB, int NB>
hipError_t launch4(const GemmWArgs& k, int nwg, hipStream_t s) {
  // K parts are planned with 2 weight blocks per tile only
  if constexpr (NB == 2) {
    if (k.KP > 1) {
      hipLaunchKernelGGL((gemmw_kernel<FMT, SWI, MB, NB, true>), dim3(nwg), dim3(64 * NWV), 0, s, k);
      return hipGetLastError();
    }
  } else {
    if (k.KP > 1) return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((gemmw_kernel<FMT, SWI, MB, NB, false>), dim3(nwg), dim3(64 * NWV), 0, s, k);
  return hipGetLastError();
}

// instantiated tile shapes: MB * NB <= 12 (accumulator registers)
template <int FMT, bool SWI, int MB>
hipError_t launch3(const GemmWArgs& k, int NB, int nwg, hipStream_t s) {
  if constexpr (MB == 1) {
    if (NB == 2) return launch4<FMT, SWI, 1, 2>(k, nwg, s);
  } else if constexpr (MB == 4) {
    if (NB == 2) return launch4<FMT, SWI, 4, 2>(k, nwg, s);
    if constexpr (!SWI) {
      if (NB == 3) return launch4<FMT, SWI, 4, 3>(k, nwg, s);
    }
  } else {
    if (NB == 2) return launch4<FMT, SWI, 2, 2>(k, nwg, s);
    if (NB == 4) return launch4<FMT, SWI, 2, 4>(k, nwg, s);
    if (NB == 6) return launch4<FMT, SWI, 2, 6>(k, nwg, s);
    if constexpr (!SWI) {
      if (NB == 3) return launch4<FMT, SWI, 2, 3>(k, nwg, s);
    }
  }
  return hipErrorInvalidValue;
}

template <int FMT, bool SWI>
hipError_t launch2(const GemmWArgs& k, const WPlan& pl, int nwg, hipStream_t s) {
  if (pl.MB == 4) return launch3<FMT, SWI, 4>(k, pl.NB, nwg, s);
  if (pl.MB == 2) return launch3<FMT, SWI, 2>(k, pl.NB, nwg, s);
  return launch3<FMT, SWI, 1>(k, pl.NB, nwg, s);
}

}  // namespace

bool gemmw_supported(const LinearArgs& a, int cus) {
  if (a.fmt != FMT_INT4 && a.fmt != FMT_INT8) return false;
  if (a.K % 32 != 0) return false;                       // whole lane halves of a K-tile
  if (gshift_of(a) < 0) return false;                    // groups: 1 per row, or 32, 64, 128, ...
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  const int64_t lim = (int64_t)1 << 31;
  if (((int64_t)(a.M - 1) * a.lda + a.K) * 2 >= lim) return false;
  if ((int64_t)a.N * a.ldw >= lim || (int64_t)a.N * a.G * 2 >= lim) return false;
  return plan(a, cus, false).ok;
}

size_t gemmw_ws_bytes(const LinearArgs& a, int cus, bool allow_split) { return plan(a, cus, allow_split).ws_bytes; }

hipError_t gemmw_launch(const LinearArgs& a, int cus, void* ws, hipStream_t s, bool allow_split) {
  const WPlan pl = plan(a, cus, allow_split);
  if (!pl.ok) return hipErrorInvalidValue;
  if (pl.KP > 1 && !ws) return hipErrorInvalidValue;
  GemmWArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.ep = a.epi_args();
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.G = a.G; k.F = a.F;
  k.gshift = gshift_of(a);
  k.BN = pl.BN; k.nbm = pl.nbm; k.nbn = pl.nbn;
  k.KT = (a.K + KTK - 1) / KTK;
  k.KP = pl.KP;
  k.tiles = pl.nbm * pl.nbn;
  if (pl.KP > 1) {
    k.cnt = (uint32_t*)ws;
    k.part = (float*)((char*)ws + kCntBytesW);
  }
  const int nwg = k.tiles * pl.KP;
  k.xcd_remap = (nwg % 8 == 0) ? 1 : 0;
  k.a_bytes = (uint32_t)(((int64_t)(a.M - 1) * a.lda + a.K) * 2);
  k.w_bytes = (uint32_t)((int64_t)a.N * a.ldw);
  // buffer loads range-check whole dwords: round up so the dword holding the
  // last entry is readable
  k.s_bytes = (uint32_t)(((int64_t)a.N * a.G * 2 + 3) & ~(int64_t)3);
  k.z_bytes = a.zeros ? k.s_bytes : 0u;
  const bool swi = a.epi == EPI_SWIGLU;
  if (a.fmt == FMT_INT4) return swi ? launch2<FMT_INT4, true>(k, pl, nwg, s) : launch2<FMT_INT4, false>(k, pl, nwg, s);
  return swi ? launch2<FMT_INT8, true>(k, pl, nwg, s) : launch2<FMT_INT8, false>(k, pl, nwg, s);
}

}  // namespace mq
