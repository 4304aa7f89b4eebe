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
// round-to-nearest-even) or an RNE conversion, or (the vector path's w / s) a
// cheaper sequence proven to give the same integer, so the result is
// bit-identical to the same steps in numpy.
//
// General path: one wavefront per (row, group), the group's elements read
// coalesced, min/max reduced across the wave, each lane writing whole bytes
// (int4: a lane owns k pairs, so g must be even).  Vector path (power-of-two
// g, aligned rows): up to 4 16-byte pieces per lane, 4- or 8-byte stores.
// HBM-bound: 2 bytes read and 0.5 (int4) or 1 (int8) byte written per weight.
#include "mq_device.hpp"
#include "mq_launch.hpp"

#pragma clang fp contract(off)

namespace mq {
namespace {

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, xor_lane(v, o));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, xor_lane(v, o));
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

// clamp(rint(x / s) + off, lo, hi) for the 8 weights of a piece, with rint of
// the IEEE quotient rounded to nearest even, at a fraction of a division's
// cost.  x and s are fp16 values, so an exact quotient that is not a
// half-integer lies at least 2^-13 from one, and the correctly rounded fp32
// quotient never lands on a half-integer it is not.  u = fma(x, fl(1/s), off)
// is within 2^-24 (|x / s| + |u|) of x / s + off: within 2^-15 for every u
// that a clamp to [0, 15] or [1, 255] can tell apart (|u|, |x / s| <= 256;
// beyond, u and x / s + off clamp to the same end), so rint(u)
// is rint(x / s) + off unless u lies within 2^-14 of a half-integer.  A lane
// with any such u takes the division for its whole piece (a wave does so about
// once in 16 for continuous data, and for every exact tie).  off is an
// integer: int4's zero point, or 128 to make int8's q a byte.
__device__ __forceinline__ void rint_quotients(const h8& v, float sf, float off, float lo, float hi, float (&q)[8]) {
  const float r = 1.0f / sf;
  float dmax = 0.f;   // largest |u - rint(u)| (exact differences, <= 0.5)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float u = __builtin_fmaf((float)v[e], r, off);
    q[e] = rintf(u);
    dmax = fmaxf(dmax, fabsf(u - q[e]));
  }
  if (dmax > 0.5f - 0x1p-14f) {
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = rintf((float)v[e] / sf) + off;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] = fminf(fmaxf(q[e], lo), hi);
}

// Vector path (g a power of two in 8..512, K and the row stride multiples of
// 8, 16-byte aligned rows): each lane takes P 16-byte pieces of 8 weights of
// one group, L = g / (8 P) lanes per group, piece i of lane l at weight
// (i L + l) 8 of the group, so each load and store instruction of a wave
// covers a contiguous run.  The per-group work (index, range reduction, scale
// and zero) is shared by 8 P weights.  The group's range is taken in fp16
// (min, max and |.| of fp16 values are exact, so equal to the fp32 ones) and
// reduced across the L lanes as one packed (min, -max) pair.
template <int FMT, int P, bool I32>
__global__ __launch_bounds__(256) void quantize_vec_kernel(QuantizeArgs p, int lshift, Div32 dg) {
  const int lane = threadIdx.x & 63;
  const int L = 1 << lshift;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t item = (wave << (6 - lshift)) + (lane >> lshift);   // (row, group)
  const bool live = item < (int64_t)p.N * p.G;
  const int64_t it = live ? item : 0;
  // n = it / G: a multiply and a shift when every item index is below 2^31
  const int n = I32 ? (int)dg.div((uint32_t)it) : (int)(it / p.G), j = (int)(it - (int64_t)n * p.G);
  const int k0 = j * p.g + (lane & (L - 1)) * 8;
  const _Float16* wr = (const _Float16*)p.W + (int64_t)n * p.ldw;
  h8 v[P];
  bool have[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    have[i] = live && k0 + i * 8 * L < p.K;
    v[i] = h8{};
    if (have[i]) v[i] = *(const h8*)(wr + k0 + i * 8 * L);
  }
  // range pair (min, -max) for int4, (-max|w|, -max|w|) for int8; +inf when empty
  h2 m = as_h2(0x7C007C00u);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if (!have[i]) continue;
    if (FMT == FMT_INT4) {
      const h2 a = __builtin_elementwise_min(v[i].s01, v[i].s23), b = __builtin_elementwise_min(v[i].s45, v[i].s67);
      const h2 c = __builtin_elementwise_max(v[i].s01, v[i].s23), d = __builtin_elementwise_max(v[i].s45, v[i].s67);
      const h2 lo2 = __builtin_elementwise_min(a, b), hi2 = __builtin_elementwise_max(c, d);
      m = __builtin_elementwise_min(
          m, (h2){__builtin_elementwise_min(lo2.x, lo2.y), -__builtin_elementwise_max(hi2.x, hi2.y)});
    } else {
      const uint32_t* u = (const uint32_t*)&v[i];
      const h2 a = __builtin_elementwise_max(as_h2(u[0] & 0x7FFF7FFFu), as_h2(u[1] & 0x7FFF7FFFu));
      const h2 b = __builtin_elementwise_max(as_h2(u[2] & 0x7FFF7FFFu), as_h2(u[3] & 0x7FFF7FFFu));
      const h2 c = __builtin_elementwise_max(a, b);
      const _Float16 h = -__builtin_elementwise_max(c.x, c.y);
      m = __builtin_elementwise_min(m, (h2){h, h});
    }
  }
  uint32_t pr = __builtin_bit_cast(uint32_t, m);
  for (int o = 1; o < L; o <<= 1)
    pr = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(as_h2(pr), as_h2((uint32_t)__float_as_int(xor_lane(__int_as_float((int)pr), o)))));
  const float lo = (float)as_h2(pr).x, hi = -(float)as_h2(pr).y;
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
  unsigned char* orow = (unsigned char*)p.out + (int64_t)n * p.ldo;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if (!have[i]) continue;
    float q[8];
    const int k = k0 + i * 8 * L;
    // whole numbers in [0, 255] go to bytes with v_cvt_pk_u8_f32 (exact)
#define PK(x, b, acc) __builtin_amdgcn_cvt_pk_u8_f32(x, b, acc)
    if (FMT == FMT_INT4) {
      rint_quotients(v[i], sf, zp, 0.f, 15.f, q);
      // even k in bytes of one word, odd k in another: nibble pairs by one shift-or
      const uint32_t ev = PK(q[6], 3, PK(q[4], 2, PK(q[2], 1, PK(q[0], 0, 0u))));
      const uint32_t od = PK(q[7], 3, PK(q[5], 2, PK(q[3], 1, PK(q[1], 0, 0u))));
      *(uint32_t*)(orow + (k >> 1)) = ev | (od << 4);
    } else {
      rint_quotients(v[i], sf, 128.f, 1.f, 255.f, q);   // q + 128, then back to two's complement
      const uint32_t w0 = PK(q[3], 3, PK(q[2], 2, PK(q[1], 1, PK(q[0], 0, 0u)))) ^ 0x80808080u;
      const uint32_t w1 = PK(q[7], 3, PK(q[6], 2, PK(q[5], 1, PK(q[4], 0, 0u)))) ^ 0x80808080u;
      *(uint2*)(orow + k) = make_uint2(w0, w1);
    }
#undef PK
  }
}

template <int FMT>
void quantize_vec_launch(const QuantizeArgs& a, int b, hipStream_t s) {
  // b = log2(g / 8); P = min(4, g / 8) pieces per lane (8 measured slower: fewer waves)
  const int64_t items = (int64_t)a.N * a.G;
  // the item index of a lane is below the grid's waves * 64 <= items + 256
  const bool i32 = items + 256 < ((int64_t)1 << 31);
  const Div32 dg = i32 ? Div32::make((uint32_t)a.G) : Div32{0u, 0};
  auto go = [&](auto k32, auto k64, int lshift) {
    const int64_t waves = (items + (64 >> lshift) - 1) / (64 >> lshift);
    hipLaunchKernelGGL(i32 ? k32 : k64, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, a, lshift, dg);
  };
  if (b >= 2) go(quantize_vec_kernel<FMT, 4, true>, quantize_vec_kernel<FMT, 4, false>, b - 2);
  else if (b == 1) go(quantize_vec_kernel<FMT, 2, true>, quantize_vec_kernel<FMT, 2, false>, 0);
  else go(quantize_vec_kernel<FMT, 1, true>, quantize_vec_kernel<FMT, 1, false>, 0);
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
    if (a.fmt == FMT_INT4) quantize_vec_launch<FMT_INT4>(a, lshift, s);
    else quantize_vec_launch<FMT_INT8>(a, lshift, s);
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
