// Decoder glue kernels for the synthetic decode step:
// residual add + RMSNorm, rotary embedding + KV-cache write, and single-token
// grouped-query attention over the cache.  They keep the decode step at a few
// launches per layer around the quantized linears; none of them is on the
// reference's quantized path (its MiniGPT example, examples/llm_generation.py,
// does these steps in numpy).  All arithmetic is fp32 on fp16 storage, with
// fp16 roundings where a PyTorch composition of the same step rounds.
#include "mq_device.hpp"
#include "mq_launch.hpp"

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

// x <- half(x + delta) (if delta); out = half(x * rsqrt(mean(x^2) + eps) * w)
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

}  // namespace

hipError_t add_rmsnorm_launch(void* x, const void* delta, const void* w, void* out, int rows, int n, float eps,
                              hipStream_t s) {
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
  hipLaunchKernelGGL(attn_partial_kernel, dim3(nsplit, H), dim3(64), 0, s, (const _Float16*)q, (const _Float16*)kc,
                     (const _Float16*)vc, pos, (float*)ws, H, KVH, D, L, scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(H), dim3(128), 0, s, (const float*)ws, (_Float16*)out, nsplit, D);
  return hipGetLastError();
}

}  // namespace mq
