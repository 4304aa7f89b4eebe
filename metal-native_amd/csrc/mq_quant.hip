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
// One wavefront per (row, group): the group's elements are read coalesced,
// min/max reduced across the wave, then each lane writes whole bytes (int4:
// a lane owns k pairs, so g must be even).  HBM-bound: 2 bytes read and 0.5
// (int4) or 1 (int8) byte written per weight.
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

}  // namespace

hipError_t quantize_launch(const QuantizeArgs& a, hipStream_t s) {
  const int64_t items = (int64_t)a.N * a.G;
  const dim3 grid((unsigned)((items + 3) / 4));
  if (a.fmt == FMT_INT4)
    hipLaunchKernelGGL(quantize_kernel<FMT_INT4>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(quantize_kernel<FMT_INT8>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace mq
