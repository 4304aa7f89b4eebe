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
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
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
  const int64_t pos = *pos_p;
  const float* cs = cos_t + pos * D;
  const float* sn = sin_t + pos * D;
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
      else kc[((int64_t)(head - H) * L + pos) * D + j] = y;
    } else {
      vc[((int64_t)(head - H - KVH) * L + pos) * D + j] = (_Float16)x;
    }
  }
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
  const int n = (int)(*pos_p) + 1;
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
  const int n = (int)(*pos_p) + 1;
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

// Rotary embedding + cache write + attention + split combine in one launch.
// Workgroup (split c, head h), lane = position, as attn_partial_d_kernel, and:
//  * q of head h is rotated here, rounded to fp16 as rope_kv stores it;
//  * the split holding position pos rotates k and takes v of the new token
//    from qkv and uses them for that position; the workgroup of the first
//    query head of each KV group writes them into the caches (no other
//    workgroup reads position pos);
//  * the split's record (m, l, o[D]) goes out with system-scope stores (the
//    splits of a head run on different XCDs), then a per-head counter elects
//    the last workgroup of the head, which combines the splits in split order
//    and resets the counter (counters start at zero, calls are stream-ordered).
template <int D>
__global__ __launch_bounds__(64) void attn_fused_d_kernel(const _Float16* qkv, const float* cos_t, const float* sin_t,
                                                           const int64_t* pos_p, _Float16* kc, _Float16* vc,
                                                           _Float16* out, float* ws, unsigned int* cnt, int H,
                                                           int KVH, int64_t L, float scale) {
  __shared__ float qs[D];
  __shared__ float knew[D], vnew[D];
  __shared__ __align__(16) _Float16 vs[kSplit * D];   // the split's V rows (fp16), position-major
  __shared__ float ps[kSplit];
  __shared__ float wgt[64];
  __shared__ unsigned int s_arrived;
  const int c = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, nsplit = gridDim.x;
  const int grp = H / KVH, kvh = h / grp;
  // K and V rows of this lane's position first: they do not depend on pos
  // (positions past it, or past the cache's end, are loaded and masked)
  const int t = c * kSplit + lane;
  const int64_t row = ((int64_t)kvh * L + min((int64_t)t, L - 1)) * D;
  h8 kv[D / 8], vv[D / 8];
#pragma unroll
  for (int j = 0; j < D / 8; ++j) kv[j] = *(const h8*)(kc + row + 8 * j);
#pragma unroll
  for (int j = 0; j < D / 8; ++j) vv[j] = *(const h8*)(vc + row + 8 * j);
  const int64_t pos = *pos_p;
  const int n = (int)pos + 1;
  const int t0 = c * kSplit;
  const float* cs = cos_t + pos * D;
  const float* sn = sin_t + pos * D;
  constexpr int HALF = D / 2;
  auto rope = [&](const _Float16* src, int j) -> _Float16 {
    const float x = (float)src[j];
    const float pair = (float)src[j < HALF ? j + HALF : j - HALF];
    const float rot = j < HALF ? -pair : pair;
    return (_Float16)(x * cs[j] + rot * sn[j]);
  };
  float* rec = ws + ((int64_t)h * nsplit + c) * (D + 2);  // [m, l, o[D]]
  auto put = [&](float* a, float v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); };
  if (t0 >= n) {
    if (lane == 0) { put(rec, -INFINITY); put(rec + 1, 0.f); }
    for (int j = lane; j < D; j += 64) put(rec + 2 + j, 0.f);
  } else {
    const bool mine = pos >= t0 && pos < t0 + kSplit;   // this split holds the new token
    const _Float16* qrow = qkv + h * D;
    const _Float16* krow = qkv + (H + kvh) * D;
    const _Float16* vsrc = qkv + (H + KVH + kvh) * D;
    for (int j = lane; j < D; j += 64) qs[j] = (float)rope(qrow, j);
    if (mine) {
      const int64_t prow = ((int64_t)kvh * L + pos) * D;
      for (int j = lane; j < D; j += 64) {
        const _Float16 kn = rope(krow, j), vn = vsrc[j];
        knew[j] = (float)kn;
        vnew[j] = (float)vn;
        if (h % grp == 0) {
          kc[prow + j] = kn;
          vc[prow + j] = vn;
        }
      }
    }
    __syncthreads();
    float acc = 0.f;
    if (mine && t == pos) {
      for (int j = 0; j < D; ++j) acc += qs[j] * knew[j];
    } else {
#pragma unroll
      for (int j = 0; j < D / 8; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += qs[8 * j + e] * (float)kv[j][e];
    }
    const float sc = t < n ? acc * scale : -INFINITY;
    const float m = wave_max(sc);
    const float p = t < n ? expf(sc - m) : 0.f;
    const float l = wave_sum(p);
    // p.V: the V rows go to LDS as fp16 (the new token's is vnew, an fp16
    // value), then each lane sums its columns over the positions in order
    ps[lane] = p;
    if (mine && t == pos) {
#pragma unroll
      for (int j = 0; j < D / 8; ++j) {
        h8 r;
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (_Float16)vnew[8 * j + e];
        *(h8*)(vs + lane * D + 8 * j) = r;
      }
    } else {
#pragma unroll
      for (int j = 0; j < D / 8; ++j) *(h8*)(vs + lane * D + 8 * j) = vv[j];
    }
    __syncthreads();
    if (D == 128) {   // lane: columns 2*lane, 2*lane + 1
      float o0 = 0.f, o1 = 0.f;
#pragma unroll 16
      for (int u = 0; u < kSplit; ++u) {
        const h2 v2 = *(const h2*)(vs + u * D + 2 * lane);
        const float pu = ps[u];
        o0 += pu * (float)v2.x;
        o1 += pu * (float)v2.y;
      }
      put(rec + 2 + 2 * lane, o0);
      put(rec + 3 + 2 * lane, o1);
    } else {
      for (int col = lane; col < D; col += 64) {
        float o = 0.f;
#pragma unroll 16
        for (int u = 0; u < kSplit; ++u) o += ps[u] * (float)vs[u * D + col];
        put(rec + 2 + col, o);
      }
    }
    if (lane == 0) { put(rec, m); put(rec + 1, l); }
  }
  // every record store has completed before the arrival is counted
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (lane == 0) s_arrived = __hip_atomic_fetch_add(cnt + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __syncthreads();
  if (s_arrived != (unsigned)(nsplit - 1)) return;
  // the last workgroup of head h: combine the splits in split order
  auto get = [&](const float* a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); };
  const float* base = ws + (int64_t)h * nsplit * (D + 2);
  const float mc = lane < nsplit ? get(base + lane * (D + 2)) : -INFINITY;
  const float lc = lane < nsplit ? get(base + lane * (D + 2) + 1) : 0.f;
  const float mm = wave_max(mc);
  const float wc = mc != -INFINITY ? expf(mc - mm) : 0.f;
  wgt[lane] = wc;   // l and o are summed in split order
  __syncthreads();
  float ll = 0.f;
  for (int cc = 0; cc < nsplit; ++cc) ll += __shfl(lc, cc) * wgt[cc];
  constexpr int CPL = D / 64;
  float o[CPL] = {};
  for (int c0 = 0; c0 < nsplit; c0 += 8) {   // eight splits' loads in flight at a time
    float v[8][CPL];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int e = 0; e < CPL; ++e)
        v[k][e] = c0 + k < nsplit ? get(base + (c0 + k) * (D + 2) + 2 + CPL * lane + e) : 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (c0 + k < nsplit)
#pragma unroll
        for (int e = 0; e < CPL; ++e) o[e] += v[k][e] * wgt[c0 + k];
  }
#pragma unroll
  for (int e = 0; e < CPL; ++e) out[h * D + CPL * lane + e] = (_Float16)(o[e] / ll);
  if (lane == 0) __hip_atomic_store(cnt + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
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
    const float v2 = __shfl_xor(v, o);
    const int i2 = __shfl_xor(i, o);
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
    // the record stores have completed before the arrival is counted
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

size_t attn_fused_workspace(int H, int D, int64_t L) {
  // per-head counters first (256-byte aligned), then the split records
  return 256 * (((size_t)H * 4 + 255) / 256) + attn_decode_workspace(H, D, L);
}

bool attn_fused_supported(int H, int D, int64_t L) {
  return H >= 1 && (D == 64 || D == 128) && (L + kSplit - 1) / kSplit <= 64;
}

hipError_t attn_fused_launch(const void* qkv, const float* cos_t, const float* sin_t, const int64_t* pos, void* kc,
                             void* vc, void* out, int H, int KVH, int D, int64_t L, float scale, void* ws,
                             hipStream_t s) {
  const int nsplit = (int)((L + kSplit - 1) / kSplit);
  unsigned int* cnt = (unsigned int*)ws;
  float* rec = (float*)((unsigned char*)ws + 256 * (((size_t)H * 4 + 255) / 256));
  if (D == 128)
    hipLaunchKernelGGL(attn_fused_d_kernel<128>, dim3(nsplit, H), dim3(64), 0, s, (const _Float16*)qkv, cos_t, sin_t,
                       pos, (_Float16*)kc, (_Float16*)vc, (_Float16*)out, rec, cnt, H, KVH, L, scale);
  else if (D == 64)
    hipLaunchKernelGGL(attn_fused_d_kernel<64>, dim3(nsplit, H), dim3(64), 0, s, (const _Float16*)qkv, cos_t, sin_t,
                       pos, (_Float16*)kc, (_Float16*)vc, (_Float16*)out, rec, cnt, H, KVH, L, scale);
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
