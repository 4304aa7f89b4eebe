// Decoder glue kernels for the synthetic decode step:
// residual add + RMSNorm, rotary embedding + KV-cache write, and single-token
// grouped-query attention over the cache.  They keep the decode step at a few
// launches per layer around the quantized linears; none of them is on the
// reference's quantized path (its MiniGPT example, examples/llm_generation.py,
// does these steps in numpy).  All arithmetic is fp32 on fp16 storage, with
// fp16 roundings where a PyTorch composition of the same step rounds.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#include <algorithm>

namespace mq {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += xor_lane(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, xor_lane(v, o));
  return v;
}
// block-wide reduction through LDS (blockDim a multiple of 64, <= 1024)
template <bool MAX>
__device__ float block_reduce(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = MAX ? wave_max(v) : wave_sum(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = MAX ? -INFINITY : 0.f;
  for (int i = 0; i < nw; ++i) r = MAX ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

// x <- half(x + delta) (if delta); out = half(x * rsqrt(mean(x^2) + eps) * w).
// Rows of up to 8 * 1024 elements, n a multiple of 8: thread t owns elements
// [8t, 8t + 8) in registers (one 16-byte load per array, one memory round
// trip, one block reduction).
__global__ __launch_bounds__(1024) void add_rmsnorm_reg_kernel(_Float16* x, const _Float16* delta, const _Float16* w,
                                                                _Float16* out, int n, float eps) {
  __shared__ float red[16];
  _Float16* xr = x + (int64_t)blockIdx.x * n;
  const _Float16* dr = delta ? delta + (int64_t)blockIdx.x * n : nullptr;
  _Float16* orow = out + (int64_t)blockIdx.x * n;
  const int i0 = 8 * threadIdx.x;
  const bool have = i0 < n;
  h8 v = {}, wv = {}, dv = {};
  if (have) {
    v = *(const h8*)(xr + i0);
    wv = *(const h8*)(w + i0);
    if (dr) dv = *(const h8*)(dr + i0);
  }
  float ss = 0.f;
  if (have) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (dr) v[e] = (_Float16)((float)v[e] + (float)dv[e]);
      const float f = (float)v[e];
      ss += f * f;
    }
    if (dr) *(h8*)(xr + i0) = v;
  }
  const float r = rsqrtf(block_reduce<false>(ss, red) / (float)n + eps);
  if (have) {
    h8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (_Float16)((float)v[e] * r * (float)wv[e]);
    *(h8*)(orow + i0) = o;
  }
}

__global__ __launch_bounds__(1024) void add_rmsnorm_kernel(_Float16* x, const _Float16* delta, const _Float16* w,
                                                            _Float16* out, int n, float eps) {
  __shared__ float red[16];
  _Float16* xr = x + (int64_t)blockIdx.x * n;
  const _Float16* dr = delta ? delta + (int64_t)blockIdx.x * n : nullptr;
  _Float16* orow = out + (int64_t)blockIdx.x * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    _Float16 v = xr[i];
    if (dr) {
      v = (_Float16)((float)v + (float)dr[i]);
      xr[i] = v;
    }
    const float f = (float)v;
    ss += f * f;
  }
  const float r = rsqrtf(block_reduce<false>(ss, red) / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) orow[i] = (_Float16)((float)xr[i] * r * (float)w[i]);
}

// qkv = [q (H*D) | k (KVH*D) | v (KVH*D)]; q_out = rope(q); cache[:, pos] = rope(k), v
__global__ __launch_bounds__(256) void rope_kv_kernel(const _Float16* qkv, const float* cos_t, const float* sin_t,
                                                       const int64_t* pos_p, _Float16* q_out, _Float16* kc,
                                                       _Float16* vc, int H, int KVH, int D, int64_t L) {
  // a position outside [0, L) writes no cache row and reads the nearest
  // table row: never an access outside the caches or the tables
  const int64_t pos = *pos_p;
  const bool in = pos >= 0 && pos < L;
  const int64_t pt = pos < 0 ? 0 : (pos < L ? pos : L - 1);
  const float* cs = cos_t + pt * D;
  const float* sn = sin_t + pt * D;
  const int half = D / 2;
  const int total = (H + 2 * KVH) * D;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const int head = e / D, j = e - head * D;
    const float x = (float)qkv[e];
    if (head < H + KVH) {
      const float pair = (float)qkv[head * D + (j < half ? j + half : j - half)];
      const float rot = j < half ? -pair : pair;
      const _Float16 y = (_Float16)(x * cs[j] + rot * sn[j]);
      if (head < H) q_out[e] = y;
      else if (in) kc[((int64_t)(head - H) * L + pos) * D + j] = y;
    } else if (in) {
      vc[((int64_t)(head - H - KVH) * L + pos) * D + j] = (_Float16)x;
    }
  }
}

// Cache positions attended to for the device position pos: 0..pos, clamped
// to the cache (a position at or past L reads no row past the cache).
__device__ __forceinline__ int positions_in_cache(int64_t pos, int64_t L) {
  return (int)(pos < 0 ? 1 : (pos < L ? pos + 1 : L));
}

// Single-token attention, split over positions (flash-decoding): workgroup
// (split c, head h) is one wave over positions [64c, 64c + 64) and writes its
// running max m, exp-sum l and unnormalised P.V to the workspace; a second
// kernel combines the splits of each head.  Many small workgroups keep enough
// loads in flight: the cache rows are read once, by ~heads * L / 64 waves.
constexpr int kSplit = 64;

__global__ __launch_bounds__(64) void attn_partial_kernel(const _Float16* q, const _Float16* kc, const _Float16* vc,
                                                           const int64_t* pos_p, float* ws, int H, int KVH, int D,
                                                           int64_t L, float scale) {
  __shared__ float qs[512];
  __shared__ float ps[kSplit];
  const int c = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int kvh = h / (H / KVH);
  const int n = positions_in_cache(*pos_p, L);
  const int t0 = c * kSplit;
  float* rec = ws + ((int64_t)h * gridDim.x + c) * (D + 2);  // [m, l, o[D]]
  if (t0 >= n) {  // split past the last position: empty record
    if (lane == 0) { rec[0] = -INFINITY; rec[1] = 0.f; }
    for (int j = lane; j < D; j += 64) rec[2 + j] = 0.f;
    return;
  }
  for (int j = lane; j < D; j += 64) qs[j] = (float)q[h * D + j];
  __syncthreads();
  // scores: lane = position (its whole K row in flight at once)
  const int t = t0 + lane;
  float s = -INFINITY;
  if (t < n) {
    const _Float16* k = kc + ((int64_t)kvh * L + t) * D;
    float acc = 0.f;
    for (int j = 0; j < D; j += 8) {
      const h8 kv = *(const h8*)(k + j);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += qs[j + e] * (float)kv[e];  // qs: same address in all lanes
    }
    s = acc * scale;
  }
  const float m = wave_max(s);
  const float p = t < n ? expf(s - m) : 0.f;
  const float l = wave_sum(p);
  ps[lane] = p;
  __syncthreads();
  // P.V: lane owns dimension pairs; the positions' V loads are independent
  const int nt = min(kSplit, n - t0);
  const _Float16* vr = vc + ((int64_t)kvh * L + t0) * D;
  for (int j = lane; 2 * j < D; j += 64) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll 16
    for (int u = 0; u < nt; ++u) {
      const h2 v2 = *(const h2*)(vr + (int64_t)u * D + 2 * j);
      a0 += ps[u] * (float)v2.x;
      a1 += ps[u] * (float)v2.y;
    }
    rec[2 + 2 * j] = a0;
    rec[2 + 2 * j + 1] = a1;
  }
  if (lane == 0) { rec[0] = m; rec[1] = l; }
}

// The same with the head dimension known at compile time (64 or 128): lane
// = position for both phases, its K and V rows loaded together up front (one
// memory round trip); p * V goes through LDS so that lanes then sum columns
// over the split's positions in position order.  Positions past pos read a
// clamped row (finite values) with weight 0.
template <int D>
__global__ __launch_bounds__(64) void attn_partial_d_kernel(const _Float16* q, const _Float16* kc, const _Float16* vc,
                                                             const int64_t* pos_p, float* ws, int H, int KVH,
                                                             int64_t L, float scale) {
  __shared__ float qs[D];
  __shared__ float pv[kSplit * (D + 1)];
  const int c = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int kvh = h / (H / KVH);
  const int n = positions_in_cache(*pos_p, L);
  const int t0 = c * kSplit;
  float* rec = ws + ((int64_t)h * gridDim.x + c) * (D + 2);  // [m, l, o[D]]
  if (t0 >= n) {
    if (lane == 0) { rec[0] = -INFINITY; rec[1] = 0.f; }
    for (int j = lane; j < D; j += 64) rec[2 + j] = 0.f;
    return;
  }
  const int t = t0 + lane;
  const int64_t row = ((int64_t)kvh * L + min((int64_t)t, L - 1)) * D;
  h8 kv[D / 8], vv[D / 8];
#pragma unroll
  for (int j = 0; j < D / 8; ++j) kv[j] = *(const h8*)(kc + row + 8 * j);
#pragma unroll
  for (int j = 0; j < D / 8; ++j) vv[j] = *(const h8*)(vc + row + 8 * j);
  for (int j = lane; j < D; j += 64) qs[j] = (float)q[h * D + j];
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < D / 8; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += qs[8 * j + e] * (float)kv[j][e];
  const float s = t < n ? acc * scale : -INFINITY;
  const float m = wave_max(s);
  const float p = t < n ? expf(s - m) : 0.f;
  const float l = wave_sum(p);
#pragma unroll
  for (int j = 0; j < D / 8; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[lane * (D + 1) + 8 * j + e] = p * (float)vv[j][e];
  __syncthreads();
  for (int col = lane; col < D; col += 64) {
    float o = 0.f;
#pragma unroll 16
    for (int u = 0; u < kSplit; ++u) o += pv[u * (D + 1) + col];
    rec[2 + col] = o;
  }
  if (lane == 0) { rec[0] = m; rec[1] = l; }
}

// One wave per head: lanes hold the splits' maxima and sums (wave
// reductions), then lane j accumulates columns j, j+64, ... over the splits.
__global__ __launch_bounds__(64) void attn_combine_wave_kernel(const float* ws, _Float16* out, int nsplit, int D) {
  __shared__ float wgt[64];
  const int h = blockIdx.x, lane = threadIdx.x;
  const float* base = ws + (int64_t)h * nsplit * (D + 2);
  const float mc = lane < nsplit ? base[lane * (D + 2)] : -INFINITY;
  const float lc = lane < nsplit ? base[lane * (D + 2) + 1] : 0.f;
  const float m = wave_max(mc);
  const float wc = mc != -INFINITY ? expf(mc - m) : 0.f;
  const float l = wave_sum(lc * wc);
  wgt[lane] = wc;
  __syncthreads();
  for (int j = lane; j < D; j += 64) {
    float a = 0.f;
#pragma unroll 4
    for (int c = 0; c < nsplit; ++c) a += base[c * (D + 2) + 2 + j] * wgt[c];
    out[h * D + j] = (_Float16)(a / l);
  }
}

__global__ __launch_bounds__(128) void attn_combine_kernel(const float* ws, _Float16* out, int nsplit, int D) {
  const int h = blockIdx.x;
  const float* base = ws + (int64_t)h * nsplit * (D + 2);
  float m = -INFINITY;
  for (int c = 0; c < nsplit; ++c) m = fmaxf(m, base[c * (D + 2)]);
  float l = 0.f;
  for (int c = 0; c < nsplit; ++c) {
    const float mc = base[c * (D + 2)];
    if (mc != -INFINITY) l += base[c * (D + 2) + 1] * expf(mc - m);
  }
  for (int j = threadIdx.x; j < D; j += blockDim.x) {
    float a = 0.f;
    for (int c = 0; c < nsplit; ++c) {
      const float mc = base[c * (D + 2)];
      if (mc != -INFINITY) a += base[c * (D + 2) + 2 + j] * expf(mc - m);
    }
    out[h * D + j] = (_Float16)(a / l);
  }
}

// Rotary embedding + cache write + attention in one launch, one workgroup per
// query head.  Wave w takes the 64-position splits w, w + NW, ...; a split's
// K and V rows are loaded coalesced (LPR = D/8 lanes per row, each lane one
// 16-byte piece of columns 8q..8q+7, RPI = 64/LPR rows per load), the next
// split's rows prefetched while the current one computes.  Scores: per-lane
// partial dot products over the piece, summed across the LPR lanes of a row
// by recursive halving (LPR - 1 shuffles for LPR rows; lane q of a row group
// ends with row q's score).  P.V: each lane weights its rows' V pieces and the
// RPI row groups are summed by shuffles.  A wave keeps a running max / exp-sum
// / P.V over its splits; the waves' partials meet through LDS, one thread per output dimension.
// q and the new k are rotated and rounded to fp16 as rope_kv stores them; the
// new token's k and v are taken from registers (its cache row is stale until
// written) and written into the caches by the workgroup of the first query
// head of each KV group (no other workgroup reads position pos).
template <int D>
__global__ __launch_bounds__(768) void attn_head_d_kernel(const _Float16* qkv, const float* cos_t, const float* sin_t,
                                                          const int64_t* pos_p, _Float16* kc, _Float16* vc,
                                                          _Float16* out, int H, int KVH, int64_t L, float scale) {
  // floating-point attention (checked against a tolerance, not bit-exact):
  // multiply-adds may fuse here, unlike in the dequant arithmetic
#pragma clang fp contract(fast)
  constexpr int LPR = D / 8;        // lanes per row
  constexpr int RPI = 64 / LPR;     // rows per load instruction
  constexpr int NI = 8;             // row loads per step (K and V: 64 VGPRs)
  constexpr int SUB = NI * RPI;     // positions per step: 32 (D = 128) or 64 (D = 64)
  constexpr int DUP = LPR / NI;     // lanes left holding the same score after the halving
  constexpr int HALF = D / 2;
  __shared__ float qs[D];
  __shared__ __align__(16) _Float16 kn16[D], vn16[D];   // the new token's rotated k and its v
  __shared__ float wm[12], wl[12], wo[12][D];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int NW = blockDim.x >> 6;
  const int q = lane % LPR, rg = lane / LPR;   // column piece, row group
  const int nsplit = (int)((L + SUB - 1) / SUB);   // steps over the cache
  const int grp = H / KVH, kvh = h / grp;
  h8 kv[NI], vv[NI];
  auto load_rows = [&](int c) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int64_t t = min((int64_t)(c * SUB + RPI * i + rg), L - 1);
      const int64_t off = ((int64_t)kvh * L + t) * D + 8 * q;
      kv[i] = *(const h8*)(kc + off);
      vv[i] = *(const h8*)(vc + off);
    }
  };
  load_rows(w);   // NW <= nsplit: every wave has a first split
  // positions outside [0, L): no cache write, attention over the cache rows
  // that exist, the nearest table row (no access outside any buffer)
  const int64_t pos = *pos_p;
  const bool in = pos >= 0 && pos < L;
  const int n = positions_in_cache(pos, L);
  const int64_t pt = pos < 0 ? 0 : (pos < L ? pos : L - 1);
  const float* cs = cos_t + pt * D;
  const float* sn = sin_t + pt * D;
  auto rope = [&](const _Float16* src, int j) -> _Float16 {
    const float x = (float)src[j];
    const float pair = (float)src[j < HALF ? j + HALF : j - HALF];
    const float rot = j < HALF ? -pair : pair;
    return (_Float16)(x * cs[j] + rot * sn[j]);
  };
  {
    const _Float16* qrow = qkv + h * D;
    const _Float16* krow = qkv + (H + kvh) * D;
    const _Float16* vsrc = qkv + (H + KVH + kvh) * D;
    const int64_t prow = ((int64_t)kvh * L + pt) * D;
    for (int j = tid; j < D; j += blockDim.x) {
      qs[j] = (float)rope(qrow, j);
      const _Float16 kn = rope(krow, j), vn = vsrc[j];
      kn16[j] = kn;
      vn16[j] = vn;
      if (in && h % grp == 0) {
        kc[prow + j] = kn;
        vc[prow + j] = vn;
      }
    }
  }
  __syncthreads();
  h2 qh[4];   // q is an fp16 value (rounded as rope_kv stores it)
#pragma unroll
  for (int e = 0; e < 4; ++e) qh[e] = (h2){(_Float16)qs[8 * q + 2 * e], (_Float16)qs[8 * q + 2 * e + 1]};
  float m_run = -INFINITY, l_run = 0.f, o_run[8] = {};
  for (int c = w; c < nsplit; c += NW) {
    const int t0 = c * SUB;
    if (t0 >= n) break;   // this and the wave's later steps lie past the new token
    if (in && pos >= t0 && pos < t0 + SUB) {   // the split holding the new token: its row from registers
      const h8 kn = *(const h8*)(kn16 + 8 * q), vn = *(const h8*)(vn16 + 8 * q);
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (t0 + RPI * i + rg == pos) { kv[i] = kn; vv[i] = vn; }
    }
    // partial scores of the lane's NI rows (row i: position t0 + RPI*i + rg)
    float d[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        a = __builtin_amdgcn_fdot2(qh[e], (h2){kv[i][2 * e], kv[i][2 * e + 1]}, a, false);
      d[i] = a;
    }
    // recursive halving across the LPR lanes of the row group (lane q ends
    // with row q / DUP), then the DUP lanes of a row add theirs
#pragma unroll
    for (int b = LPR / 2, S = NI; S > 1; b >>= 1, S >>= 1) {
      const bool up = (q & b) != 0;
#pragma unroll
      for (int k = 0; k < S / 2; ++k) {
        const float keep = up ? d[k + S / 2] : d[k];
        const float send = up ? d[k] : d[k + S / 2];
        d[k] = keep + xor_lane(send, b);
      }
    }
#pragma unroll
    for (int b = DUP / 2; b >= 1; b >>= 1) d[0] += xor_lane(d[0], b);
    const int t = t0 + RPI * (q / DUP) + rg;   // the position whose full score this lane holds
    const float sc = t < n ? d[0] * scale : -INFINITY;
    const float m = wave_max(sc);
    const float p = t < n ? expf(sc - m) : 0.f;
    const float l = wave_sum(q % DUP == 0 ? p : 0.f);
    float o[8] = {};
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float pi;   // p of row i of this row group: lane i * DUP of it
      if constexpr (LPR == 16)
        pi = row_bcast(p, i * DUP);
      else
        pi = __shfl(p, rg * LPR + i * DUP);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += pi * (float)vv[i][e];
    }
    // the next split's rows: issued once this split's are consumed (the fence
    // keeps the loads from being hoisted above the uses, doubling the rows live)
    asm volatile("" ::: "memory");
    if (c + NW < nsplit) load_rows(c + NW);
#pragma unroll
    for (int b = LPR; b < 64; b <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += xor_lane(o[e], b);
    const float mn = fmaxf(m_run, m);
    const float a = m_run == -INFINITY ? 0.f : expf(m_run - mn), bsc = expf(m - mn);
    l_run = l_run * a + l * bsc;
#pragma unroll
    for (int e = 0; e < 8; ++e) o_run[e] = o_run[e] * a + o[e] * bsc;
    m_run = mn;
  }
  if (lane == 0) { wm[w] = m_run; wl[w] = l_run; }
  if (rg == 0)
#pragma unroll
    for (int e = 0; e < 8; ++e) wo[w][8 * q + e] = o_run[e];
  __syncthreads();
  // the waves' partials meet in wave order, one thread per output dimension
  if (tid < D) {
    float mm = -INFINITY;
    for (int ww = 0; ww < NW; ++ww) mm = fmaxf(mm, wm[ww]);
    float ll = 0.f, o = 0.f;
    for (int ww = 0; ww < NW; ++ww) {
      const float f = wm[ww] == -INFINITY ? 0.f : expf(wm[ww] - mm);
      ll += wl[ww] * f;
      o += wo[ww][tid] * f;
    }
    out[h * D + tid] = (_Float16)(o / ll);
  }
}

// ---- greedy decode tail: token = argmax(logits), pos += 1, x = embed[token] ----
// torch.argmax order: NaN above every number, ties to the lowest index.
__device__ __forceinline__ bool am_better(float v1, int i1, float v2, int i2) {
  const bool n1 = v1 != v1, n2 = v2 != v2;
  if (n1 != n2) return n1;
  if (!n1 && v1 != v2) return v1 > v2;
  return i1 < i2;
}
__device__ __forceinline__ void am_wave(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = xor_lane(v, o);
    const int i2 = __float_as_int(xor_lane(__int_as_float(i), o));
    if (am_better(v2, i2, v, i)) { v = v2; i = i2; }
  }
}
// 256 threads x 8 logits per workgroup; the per-workgroup best goes to a
// record (system-scope stores), and the last workgroup to arrive reduces the
// records, writes the token and the next position and copies the embedding
// row, then clears the arrival counter for the next launch.
__global__ __launch_bounds__(256) void argmax_embed_kernel(const _Float16* logits, int V, const _Float16* embed,
                                                           int64_t lde, int d, int64_t* tok, int64_t* pos,
                                                           _Float16* x, float* rv, int* ri, unsigned* cnt) {
  __shared__ float sv[4];
  __shared__ int si[4];
  __shared__ unsigned s_arrived;
  __shared__ int s_tok;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int nwg = gridDim.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const int i0 = (blockIdx.x * 256 + t) * 8;
  if (i0 + 8 <= V && ((uintptr_t)logits & 15) == 0) {
    const h8 v = *(const h8*)(logits + i0);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (am_better((float)v[e], i0 + e, bv, bi)) { bv = (float)v[e]; bi = i0 + e; }
  } else {
    for (int e = 0; e < 8 && i0 + e < V; ++e) {
      const float f = (float)logits[i0 + e];
      if (am_better(f, i0 + e, bv, bi)) { bv = f; bi = i0 + e; }
    }
  }
  am_wave(bv, bi);
  if (lane == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  if (t == 0) {
    for (int k = 1; k < 4; ++k)
      if (am_better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
    __hip_atomic_store(rv + blockIdx.x, bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(ri + blockIdx.x, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    // the record stores (system-scope atomics, written through to memory)
    // are acknowledged before the arrival is counted; the last arriver reads
    // them with system-scope atomic loads: a release/acquire pair without
    // the L2 writeback/invalidate, which only non-atomic accesses would need
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    s_arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  __syncthreads();
  if (s_arrived != (unsigned)(nwg - 1)) return;
  bv = -INFINITY;
  bi = 0x7fffffff;
  for (int k = t; k < nwg; k += 256) {
    const float v2 = __hip_atomic_load(rv + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int i2 = __hip_atomic_load(ri + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (am_better(v2, i2, bv, bi)) { bv = v2; bi = i2; }
  }
  am_wave(bv, bi);
  if (lane == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  if (t == 0) {
    for (int k = 1; k < 4; ++k)
      if (am_better(sv[k], si[k], bv, bi)) { bv = sv[k]; bi = si[k]; }
    s_tok = bi;
    tok[0] = bi;
    pos[0] = pos[0] + 1;
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  __syncthreads();
  const _Float16* row = embed + (int64_t)s_tok * lde;
  for (int k = t; k < d; k += 256) x[k] = row[k];
}

}  // namespace

hipError_t add_rmsnorm_launch(void* x, const void* delta, const void* w, void* out, int rows, int n, float eps,
                              hipStream_t s) {
  if (n <= 8 * 1024 && n % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
      ((uintptr_t)out & 15) == 0 && ((uintptr_t)delta & 15) == 0) {
    const int nt = std::min(1024, (n / 8 + 63) / 64 * 64);
    hipLaunchKernelGGL(add_rmsnorm_reg_kernel, dim3(rows), dim3(nt), 0, s, (_Float16*)x, (const _Float16*)delta,
                       (const _Float16*)w, (_Float16*)out, n, eps);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(rows), dim3(1024), 0, s, (_Float16*)x, (const _Float16*)delta,
                     (const _Float16*)w, (_Float16*)out, n, eps);
  return hipGetLastError();
}

hipError_t rope_kv_launch(const void* qkv, const float* cos_t, const float* sin_t, const int64_t* pos, void* q_out,
                          void* kc, void* vc, int H, int KVH, int D, int64_t L, hipStream_t s) {
  const int total = (H + 2 * KVH) * D;
  hipLaunchKernelGGL(rope_kv_kernel, dim3((total + 255) / 256), dim3(256), 0, s, (const _Float16*)qkv, cos_t, sin_t,
                     pos, (_Float16*)q_out, (_Float16*)kc, (_Float16*)vc, H, KVH, D, L);
  return hipGetLastError();
}

size_t attn_decode_workspace(int H, int D, int64_t L) {
  return (size_t)H * ((L + kSplit - 1) / kSplit) * (D + 2) * sizeof(float);
}

hipError_t attn_decode_launch(const void* q, const void* kc, const void* vc, const int64_t* pos, void* out, int H,
                              int KVH, int D, int64_t L, float scale, void* ws, hipStream_t s) {
  const int nsplit = (int)((L + kSplit - 1) / kSplit);
  if (D == 128)
    hipLaunchKernelGGL(attn_partial_d_kernel<128>, dim3(nsplit, H), dim3(64), 0, s, (const _Float16*)q,
                       (const _Float16*)kc, (const _Float16*)vc, pos, (float*)ws, H, KVH, L, scale);
  else if (D == 64)
    hipLaunchKernelGGL(attn_partial_d_kernel<64>, dim3(nsplit, H), dim3(64), 0, s, (const _Float16*)q,
                       (const _Float16*)kc, (const _Float16*)vc, pos, (float*)ws, H, KVH, L, scale);
  else
    hipLaunchKernelGGL(attn_partial_kernel, dim3(nsplit, H), dim3(64), 0, s, (const _Float16*)q, (const _Float16*)kc,
                       (const _Float16*)vc, pos, (float*)ws, H, KVH, D, L, scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (nsplit <= 64)
    hipLaunchKernelGGL(attn_combine_wave_kernel, dim3(H), dim3(64), 0, s, (const float*)ws, (_Float16*)out, nsplit, D);
  else
    hipLaunchKernelGGL(attn_combine_kernel, dim3(H), dim3(128), 0, s, (const float*)ws, (_Float16*)out, nsplit, D);
  return hipGetLastError();
}

bool attn_fused_supported(int H, int D, int64_t L) {
  return H >= 1 && (D == 64 || D == 128) && (L + kSplit - 1) / kSplit <= 64;
}

hipError_t attn_fused_launch(const void* qkv, const float* cos_t, const float* sin_t, const int64_t* pos, void* kc,
                             void* vc, void* out, int H, int KVH, int D, int64_t L, float scale, hipStream_t s) {
  const int NW = std::min<int64_t>(12, (L + 4095 / D) / (4096 / D));   // one wave per step up to 12
  if (D == 128)
    hipLaunchKernelGGL(attn_head_d_kernel<128>, dim3(H), dim3(64 * NW), 0, s, (const _Float16*)qkv, cos_t, sin_t,
                       pos, (_Float16*)kc, (_Float16*)vc, (_Float16*)out, H, KVH, L, scale);
  else if (D == 64)
    hipLaunchKernelGGL(attn_head_d_kernel<64>, dim3(H), dim3(64 * NW), 0, s, (const _Float16*)qkv, cos_t, sin_t,
                       pos, (_Float16*)kc, (_Float16*)vc, (_Float16*)out, H, KVH, L, scale);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

size_t argmax_embed_workspace(int64_t V) {
  const int64_t nwg = (V + 2047) / 2048;
  return 256 + 8 * (size_t)nwg;   // counter (256-byte aligned), then values and indices
}

hipError_t argmax_embed_launch(const void* logits, int64_t V, const void* embed, int64_t lde, int d, int64_t* tok,
                               int64_t* pos, void* x, void* ws, hipStream_t s) {
  const int nwg = (int)((V + 2047) / 2048);
  unsigned* cnt = (unsigned*)ws;
  float* rv = (float*)((unsigned char*)ws + 256);
  int* ri = (int*)(rv + nwg);
  hipLaunchKernelGGL(argmax_embed_kernel, dim3(nwg), dim3(256), 0, s, (const _Float16*)logits, (int)V,
                     (const _Float16*)embed, lde, d, tok, pos, (_Float16*)x, rv, ri, cnt);
  return hipGetLastError();
}

}  // namespace mq
