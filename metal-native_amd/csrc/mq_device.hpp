// Device-side building blocks for the quantized-linear kernels (gfx950 only).
//
// Storage formats are the reference's (kimsejun0629/metal-native):
//   int4: uint8 [N, K/2], byte j of row n = (k=2j low nibble, k=2j+1 high
//         nibble)  -- shaders/matmul_dequant_kernel.metal:37-38,129-139
//   int8: int8  [N, K]                    -- matmul_dequant_kernel.metal:400-412
//   scales/zeros: fp16 [N, ceil(K/g)], group of k is k/g  -- :98,141-143
// Dequant: w = half(q-8)*s - z (int4), w = half(q)*s - z (int8), two fp16
// roundings, multiply first (matmul_dequant_kernel.metal:42-43,47-49).
//
// Every translation unit that includes this header disables floating-point
// contraction so that the multiply and the subtract of the dequant formula are
// never fused into one FMA (which would round once instead of twice).
#pragma once
#pragma clang fp contract(off)

// gfx950 only: the cross-workgroup handoffs (split-K GEMV, K-split GEMM,
// row-block K parts, argmax) publish with relaxed system-scope atomics and
// s_waitcnt, an ordering argument made for gfx950's lowering of the memory
// model; the inline-asm MFMA code assumes gfx950's operand layouts.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the metal-native_amd kernels are written for gfx950 only"
#endif

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq_launch.hpp"

namespace mq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));


// k values covered by one 16-byte load of a weight row.
template <int FMT> struct FmtTraits;
template <> struct FmtTraits<FMT_INT4> { static constexpr int KPL = 32; };
template <> struct FmtTraits<FMT_INT8> { static constexpr int KPL = 16; };
template <> struct FmtTraits<FMT_F16>  { static constexpr int KPL = 8; };

// Cross-lane exchanges without the LDS unit: within 16-lane rows by DPP
// (quad_perm, row_mirror 0x140, row_half_mirror 0x141), across rows by the
// permlane swaps.  xor_lane(v, b) is v of lane (lane ^ b), b a power of two
// known after unrolling.
__device__ __forceinline__ int dpp_(int x, int ctrl) {
  switch (ctrl) {   // the control must be a constant of the instruction
    case 0xB1: return __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    case 0x4E: return __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    case 0x1B: return __builtin_amdgcn_update_dpp(0, x, 0x1B, 0xF, 0xF, false);   // quad_perm [3,2,1,0]
    case 0x140: return __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false); // row_mirror: ^15
    default: return __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);    // row_half_mirror: ^7
  }
}
// v of lane n of the lane's 16-lane row (DPP row_newbcast)
__device__ __forceinline__ float row_bcast(float v, int n) {
  const int x = __float_as_int(v);
#define RB(k) \
  case k: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x150 + k, 0xF, 0xF, false));
  switch (n) {
    RB(0) RB(1) RB(2) RB(3) RB(4) RB(5) RB(6) RB(7) RB(8) RB(9) RB(10) RB(11) RB(12) RB(13) RB(14)
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x15F, 0xF, 0xF, false));
  }
#undef RB
}
__device__ __forceinline__ float xor_lane(float v, int b) {
  const int x = __float_as_int(v);
  const bool hi = (threadIdx.x & b) != 0;
  switch (b) {
    case 1: return __int_as_float(dpp_(x, 0xB1));
    case 2: return __int_as_float(dpp_(x, 0x4E));
    case 4: return __int_as_float(dpp_(dpp_(x, 0x141), 0x1B));    // (^7) then (^3)
    case 8: return __int_as_float(dpp_(dpp_(x, 0x140), 0x141));   // (^15) then (^7)
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);   // rows (0,0,2,2), (1,1,3,3)
      return __int_as_float(hi ? (int)r[0] : (int)r[1]);
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);   // halves (0,0), (1,1)
      return __int_as_float(hi ? (int)r[0] : (int)r[1]);
    }
  }
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Exact fp16 "q - 8" for two nibbles placed at bits [3:0] and [19:16]:
// 0x6400 is 1024.0, so OR-ing a nibble into the low mantissa bits gives 1024+q
// exactly, and subtracting 1032 gives q-8 exactly.
__device__ __forceinline__ h2 nib_lo_pair(uint32_t d) {
  return as_h2((d & 0x000F000Fu) | 0x64006400u) - (h2){(_Float16)1032.0f, (_Float16)1032.0f};
}
// Same for nibbles at bits [7:4] and [23:20]: the halves hold 1024+16q, and
// (1024+16q)/16 - 72 = q-8.  Every intermediate is exact, so a fused
// multiply-add is used deliberately here.
__device__ __forceinline__ h2 nib_hi_pair(uint32_t d) {
  h2 v = as_h2((d & 0x00F000F0u) | 0x64006400u);
  return __builtin_elementwise_fma(v, (h2){(_Float16)0.0625f, (_Float16)0.0625f},
                                   (h2){(_Float16)-72.0f, (_Float16)-72.0f});
}

// w = RNE(RNE(q*s) - z): one packed multiply and one packed subtract.
__device__ __forceinline__ h2 scale_sub(h2 q, h2 s, h2 z) {
  h2 t = q * s;
  return t - z;
}

// Eight int4 weights of one dword (k0..k7 at bits 4i) dequantized into the
// MFMA-operand order [k0,k4,k1,k5,k2,k6,k3,k7].  Activations multiplied
// against these are staged in the same order (see perm8_int4).
__device__ __forceinline__ h8 dq_int4_dword_perm(uint32_t d, h2 s, h2 z) {
  uint32_t d8 = d >> 8;
  h2 p0 = scale_sub(nib_lo_pair(d), s, z);   // k0, k4
  h2 p1 = scale_sub(nib_hi_pair(d), s, z);   // k1, k5
  h2 p2 = scale_sub(nib_lo_pair(d8), s, z);  // k2, k6
  h2 p3 = scale_sub(nib_hi_pair(d8), s, z);  // k3, k7
  h8 r;
  r.s01 = p0; r.s23 = p1; r.s45 = p2; r.s67 = p3;
  return r;
}

// Same as dq_int4_dword_perm with the masks and the 0x6400 pair passed in as
// values: kept in registers they let the compiler emit one v_and_or_b32 per
// nibble pair instead of an AND and an OR with literal operands.
// (d & mask) | magic in one VALU op; mask lives in a VGPR and magic in an SGPR
// (gfx9 VOP3 encodings take one scalar operand and no literal).
__device__ __forceinline__ uint32_t and_or(uint32_t d, uint32_t mask_v, uint32_t magic_s) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(d), "v"(mask_v), "s"(magic_s));
  return r;
}
__device__ __forceinline__ h8 dq_int4_dword_perm_r(uint32_t d, h2 s, h2 z, uint32_t mlo, uint32_t mhi,
                                                   uint32_t magic) {
  const uint32_t d8 = d >> 8;
  const h2 c1032 = (h2){(_Float16)1032.0f, (_Float16)1032.0f};
  const h2 c16 = (h2){(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 c72 = (h2){(_Float16)-72.0f, (_Float16)-72.0f};
  h8 r;
  r.s01 = scale_sub(as_h2(and_or(d, mlo, magic)) - c1032, s, z);                                // k0, k4
  r.s23 = scale_sub(__builtin_elementwise_fma(as_h2(and_or(d, mhi, magic)), c16, c72), s, z);   // k1, k5
  r.s45 = scale_sub(as_h2(and_or(d8, mlo, magic)) - c1032, s, z);                               // k2, k6
  r.s67 = scale_sub(__builtin_elementwise_fma(as_h2(and_or(d8, mhi, magic)), c16, c72), s, z);  // k3, k7
  return r;
}

// Eight int4 weights in natural k order (used where the output is stored,
// i.e. the dequantize op).  v_perm_b32 copies byte b into bytes 0 and 2 so
// the two nibbles of one byte land in the two fp16 halves.
__device__ __forceinline__ h2 nib_byte_pair(uint32_t d, uint32_t sel) {
  uint32_t e = __builtin_amdgcn_perm(0u, d, sel);  // bytes [b, 0, b, 0]
  h2 v = as_h2((e & 0x00F0000Fu) | 0x64006400u);   // (1024+lo, 1024+16*hi)
  return __builtin_elementwise_fma(v, (h2){(_Float16)1.0f, (_Float16)0.0625f},
                                   (h2){(_Float16)-1032.0f, (_Float16)-72.0f});
}
// Natural-order variant with the nibble mask in a VGPR and the 0x6400 pair
// in an SGPR: one v_and_or_b32 per pair instead of an AND and an OR with
// literal operands (five VALU ops per pair of weights).
__device__ __forceinline__ h8 dq_int4_dword_nat_r(uint32_t d, h2 s, h2 z, uint32_t mask_v, uint32_t magic_s) {
  const h2 m = (h2){(_Float16)1.0f, (_Float16)0.0625f};
  const h2 o = (h2){(_Float16)-1032.0f, (_Float16)-72.0f};
  h8 r;
  r.s01 = scale_sub(__builtin_elementwise_fma(as_h2(and_or(__builtin_amdgcn_perm(0u, d, 0x0c000c00u), mask_v, magic_s)), m, o), s, z);
  r.s23 = scale_sub(__builtin_elementwise_fma(as_h2(and_or(__builtin_amdgcn_perm(0u, d, 0x0c010c01u), mask_v, magic_s)), m, o), s, z);
  r.s45 = scale_sub(__builtin_elementwise_fma(as_h2(and_or(__builtin_amdgcn_perm(0u, d, 0x0c020c02u), mask_v, magic_s)), m, o), s, z);
  r.s67 = scale_sub(__builtin_elementwise_fma(as_h2(and_or(__builtin_amdgcn_perm(0u, d, 0x0c030c03u), mask_v, magic_s)), m, o), s, z);
  return r;
}
__device__ __forceinline__ h8 dq_int4_dword_nat(uint32_t d, h2 s, h2 z) {
  h8 r;
  r.s01 = scale_sub(nib_byte_pair(d, 0x0c000c00u), s, z);
  r.s23 = scale_sub(nib_byte_pair(d, 0x0c010c01u), s, z);
  r.s45 = scale_sub(nib_byte_pair(d, 0x0c020c02u), s, z);
  r.s67 = scale_sub(nib_byte_pair(d, 0x0c030c03u), s, z);
  return r;
}

// Four int8 weights of one dword in natural order.  XOR 0x80 turns the signed
// byte q into q+128 (0..255); v_perm_b32 places it under a 0x64 high byte,
// giving fp16 1024+q+128 exactly; subtracting 1152 gives q exactly.
__device__ __forceinline__ void dq_int8_dword(uint32_t d, h2 s, h2 z, h2& lo, h2& hi) {
  uint32_t u = d ^ 0x80808080u;
  const h2 off = (h2){(_Float16)1152.0f, (_Float16)1152.0f};
  h2 q01 = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - off;
  h2 q23 = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - off;
  lo = scale_sub(q01, s, z);
  hi = scale_sub(q23, s, z);
}

// Reorder eight fp16 activations (natural k order, as four dwords) into the
// int4 operand order [x0,x4,x1,x5,x2,x6,x3,x7].
__device__ __forceinline__ u4 perm8_int4(u4 v) {
  u4 r;
  r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);  // x0 | x4<<16
  r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);  // x1 | x5<<16
  r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);  // x2 | x6<<16
  r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);  // x3 | x7<<16
  return r;
}

__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Read-out fence for MFMA accumulators: 24 wait states with the accumulator
// as an in/out operand, so the MFMA that wrote it has retired before any
// VALU/LDS/VMEM instruction reads it.  A guard, not a fix the current
// compiler needs: an early split-K fold read stale upper accumulator
// registers with the compiler's own padding (about 8 wait states after a
// v_mfma_f32_16x16x32_f16), and the whole GPU test suite also passes with
// this fence compiled out under ROCm 7.2 (clang 22).  It costs 24 cycles per
// accumulator read-out (once per tile), and every read-out of an MFMA result
// in this library goes through it (mq_gemmw.hip spells it with AGPR operands).
__device__ __forceinline__ void mfma_result_fence(f4& v) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(v));
}

// ---- buffer loads ----
// A buffer load whose offset lies outside the descriptor's range returns
// zeros without touching memory; kOob is such an offset for every range used
// here (all ranges are below 2^31 bytes).  Loads issued unconditionally this
// way keep the compiler's load counter exact.
constexpr uint32_t kOob = 0x80000000u;
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u4 bload16_nt(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
__device__ __forceinline__ uint64_t bload8_nt(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2));
}
__device__ __forceinline__ u4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint16_t bload2h(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// 8 halves of padding after every 128 activations: the K shifts and lane
// groups of one wave read fall in different LDS banks.
__device__ __forceinline__ int xswz(int k) { return k + ((k >> 7) << 3); }


__device__ __forceinline__ void mfma_result_fence16(f16v& v) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(v));
}

__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

// Element-wise epilogue on the fp32 accumulator of output (row, col), before
// the one fp16 rounding (shaders/matmul_fused_epilogue.metal:97-124): bias
// add, bias + ReLU, bias + SiLU v/(1+exp(-v)), residual add.  The switch is
// on a kernel argument (uniform), outside the K loop.
__device__ __forceinline__ float epi_apply(float v, int64_t row, int col, const EpiArgs& e) {
  switch (e.epi) {
    case EPI_BIAS: return v + (float)((const _Float16*)e.bias)[col];
    case EPI_BIAS_RELU: return fmaxf(v + (float)((const _Float16*)e.bias)[col], 0.0f);
    case EPI_BIAS_SILU: return silu_f32(v + (float)((const _Float16*)e.bias)[col]);
    case EPI_RESIDUAL: return v + (float)((const _Float16*)e.resid)[row * e.ldr + col];
    default: return v;
  }
}

// Scalar dequant of one element (generic kernels).
__device__ __forceinline__ _Float16 dq_scalar(int q, _Float16 s, _Float16 z) {
  _Float16 qh = (_Float16)q;
  _Float16 t = qh * s;
  return t - z;
}

}  // namespace mq
