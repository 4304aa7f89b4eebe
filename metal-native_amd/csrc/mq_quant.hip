// Group quantizer: fp16 W [N, K] -> the reference's storage format
// (int4 [N, K/2] nibble pairs or int8 [N, K], fp16 scales/zeros [N, G]).
//
// The reference has no quantizer (its tests pack by hand,
// tests/cpp/test_dequant_matmul.mm:104-116); this is the inverse of its
// dequant formula w = half(q - 8) * s - z (shaders/matmul_dequant_kernel.metal:29-49):
//   int4, asymmetric per group: s = half((max - min) / 15) (1 when 0),
//     zp = clamp(rint(-min / s), 0, 15), q = clamp(rint(w / s) + zp, 0, 15),
//     z = half((zp - 8) * s), so that (q - 8) * s - z ~= (q - zp) * s;
//   int8, symmetric per group: s = half(max|w| / 127) (1 when 0),
//     q = clamp(rint(w / s), -127, 127), z = 0.
// Every step is one IEEE fp32 operation (min/max, correctly rounded division,
// round-to-nearest-even) or an RNE conversion, so the result is bit-identical
// to the same steps in numpy.
//
// General path: one wavefront per (row, group), the group's elements read
// coalesced, min/max reduced across the wave, each lane writing whole bytes
// (int4: a lane owns k pairs, so g must be even).  Vector path (power-of-two
// g, aligned rows): g/8 lanes per group, 16-byte loads, 4- or 8-byte stores.
// HBM-bound: 2 bytes read and 0.5 (int4) or 1 (int8) byte written per weight.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#pragma clang fp contract(off)

namespace mq {
namespace {

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

template <int FMT>
__global__ __launch_bounds__(256) void quantize_kernel(QuantizeArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (row, group)
  if (item >= (int64_t)p.N * p.G) return;
  const int n = (int)(item / p.G), j = (int)(item - (int64_t)n * p.G);
  const int k0 = j * p.g, k1 = min(p.K, k0 + p.g);
  const _Float16* wr = (const _Float16*)p.W + (int64_t)n * p.ldw;

  float lo = INFINITY, hi = -INFINITY;
  if (FMT == FMT_INT4) {
    for (int k = k0 + 2 * lane; k < k1; k += 128) {   // k even, k + 1 < k1 (g and K even)
      const h2 v = *(const h2*)(wr + k);
      const float a = (float)v.x, b = (float)v.y;
      lo = fminf(lo, fminf(a, b));
      hi = fmaxf(hi, fmaxf(a, b));
    }
  } else {
    for (int k = k0 + lane; k < k1; k += 64) hi = fmaxf(hi, fabsf((float)wr[k]));
  }
  hi = wave_max(hi);
  float sf, zp = 0.f;
  _Float16 s16, z16 = (_Float16)0.f;
  if (FMT == FMT_INT4) {
    lo = wave_min(lo);
    s16 = (_Float16)((hi - lo) / 15.0f);
    if (s16 == (_Float16)0.f) s16 = (_Float16)1.f;
    sf = (float)s16;
    zp = fminf(fmaxf(rintf(-lo / sf), 0.f), 15.f);
    z16 = (_Float16)((zp - 8.0f) * sf);
  } else {
    s16 = (_Float16)(hi / 127.0f);
    if (s16 == (_Float16)0.f) s16 = (_Float16)1.f;
    sf = (float)s16;
  }
  if (lane == 0) {
    ((_Float16*)p.scales)[(int64_t)n * p.G + j] = s16;
    ((_Float16*)p.zeros)[(int64_t)n * p.G + j] = z16;
  }
  if (FMT == FMT_INT4) {
    unsigned char* out = (unsigned char*)p.out + (int64_t)n * p.ldo;
    for (int k = k0 + 2 * lane; k < k1; k += 128) {
      const h2 v = *(const h2*)(wr + k);
      const float qa = fminf(fmaxf(rintf((float)v.x / sf) + zp, 0.f), 15.f);
      const float qb = fminf(fmaxf(rintf((float)v.y / sf) + zp, 0.f), 15.f);
      out[k >> 1] = (unsigned char)((int)qa | ((int)qb << 4));
    }
  } else {
    signed char* out = (signed char*)p.out + (int64_t)n * p.ldo;
    for (int k = k0 + lane; k < k1; k += 64)
      out[k] = (signed char)(int)fminf(fmaxf(rintf((float)wr[k] / sf), -127.f), 127.f);
  }
}

// Vector path (g a power of two in 8..512, K and the row stride multiples of
// 8, 16-byte aligned rows): L = g/8 lanes per group, each lane one 16-byte
// piece of 8 weights; a wave covers 64/L groups.  Same arithmetic as above.
template <int FMT>
__global__ __launch_bounds__(256) void quantize_vec_kernel(QuantizeArgs p, int lshift) {
  const int lane = threadIdx.x & 63;
  const int L = 1 << lshift;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t item = (wave << (6 - lshift)) + (lane >> lshift);   // (row, group)
  const bool live = item < (int64_t)p.N * p.G;
  const int64_t it = live ? item : 0;
  const int n = (int)(it / p.G), j = (int)(it - (int64_t)n * p.G);
  const int k = j * p.g + (lane & (L - 1)) * 8;
  const bool have = live && k < p.K;
  h8 v = {};
  if (have) v = *(const h8*)((const _Float16*)p.W + (int64_t)n * p.ldw + k);
  float lo = INFINITY, hi = -INFINITY;
  if (have) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = (float)v[e];
      if (FMT == FMT_INT4) {
        lo = fminf(lo, f);
        hi = fmaxf(hi, f);
      } else {
        hi = fmaxf(hi, fabsf(f));
      }
    }
  }
  for (int o = 1; o < L; o <<= 1) {
    hi = fmaxf(hi, __shfl_xor(hi, o));
    if (FMT == FMT_INT4) lo = fminf(lo, __shfl_xor(lo, o));
  }
  float sf, zp = 0.f;
  _Float16 s16, z16 = (_Float16)0.f;
  if (FMT == FMT_INT4) {
    s16 = (_Float16)((hi - lo) / 15.0f);
    if (s16 == (_Float16)0.f) s16 = (_Float16)1.f;
    sf = (float)s16;
    zp = fminf(fmaxf(rintf(-lo / sf), 0.f), 15.f);
    z16 = (_Float16)((zp - 8.0f) * sf);
  } else {
    s16 = (_Float16)(hi / 127.0f);
    if (s16 == (_Float16)0.f) s16 = (_Float16)1.f;
    sf = (float)s16;
  }
  if (live && (lane & (L - 1)) == 0) {
    ((_Float16*)p.scales)[it] = s16;   // [N, G] contiguous: index n*G + j
    ((_Float16*)p.zeros)[it] = z16;
  }
  if (!have) return;
  if (FMT == FMT_INT4) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = fminf(fmaxf(rintf((float)v[e] / sf) + zp, 0.f), 15.f);
      word |= (uint32_t)(int)q << (4 * e);
    }
    *(uint32_t*)((unsigned char*)p.out + (int64_t)n * p.ldo + (k >> 1)) = word;
  } else {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int q = (int)fminf(fmaxf(rintf((float)v[e] / sf), -127.f), 127.f);
      if (e < 4) w0 |= (uint32_t)(q & 0xFF) << (8 * e);
      else w1 |= (uint32_t)(q & 0xFF) << (8 * (e - 4));
    }
    *(uint2*)((unsigned char*)p.out + (int64_t)n * p.ldo + k) = make_uint2(w0, w1);
  }
}

}  // namespace

hipError_t quantize_launch(const QuantizeArgs& a, hipStream_t s) {
  const int64_t items = (int64_t)a.N * a.G;
  int lshift = -1;
  for (int b = 0; b <= 6; ++b)
    if (a.g == 8 << b) lshift = b;
  const bool vec = lshift >= 0 && a.K % 8 == 0 && a.ldw % 8 == 0 && ((uintptr_t)a.W & 15) == 0 &&
                   (a.fmt == FMT_INT4 ? (a.ldo % 4 == 0 && ((uintptr_t)a.out & 3) == 0)
                                      : (a.ldo % 8 == 0 && ((uintptr_t)a.out & 7) == 0));
  if (vec) {
    const int64_t waves = (items + (64 >> lshift) - 1) / (64 >> lshift);
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (a.fmt == FMT_INT4)
      hipLaunchKernelGGL(quantize_vec_kernel<FMT_INT4>, grid, dim3(256), 0, s, a, lshift);
    else
      hipLaunchKernelGGL(quantize_vec_kernel<FMT_INT8>, grid, dim3(256), 0, s, a, lshift);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((items + 3) / 4));
  if (a.fmt == FMT_INT4)
    hipLaunchKernelGGL(quantize_kernel<FMT_INT4>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(quantize_kernel<FMT_INT8>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace mq
