// Tiled MFMA GEMM with in-LDS dequantization (prefill, M > 64).
//
// Replaces dequant_matmul_int4_fp16 / dequant_matmul_int8_fp16
// (shaders/matmul_dequant_kernel.metal:55-223, :351-479; dispatched at
// src/ops/matmul.mm:1011-1021).  Same contract: C = A . deq(W)^T with fp16
// products accumulated in fp32 and one rounding to fp16.
//
// Tile: 128 (M) x 128 (weight rows) x 32 (K) per workgroup of 4 wavefronts
// arranged 2 x 2; each wave owns a 64 x 64 sub-tile = 4 x 4 blocks of
// v_mfma_f32_16x16x32_f16.  Per K step every thread loads 32 bytes of A and
// 8 (int4) or 16 (int8) bytes of W for the next step into registers while the
// current step's MFMAs run (register prefetch), then dequantizes W into an fp16
// LDS tile.  LDS holds two tile buffers so one barrier per K step suffices.
// For SwiGLU the 128 weight rows are 64 gate rows and the matching 64 up rows,
// and the output tile is 128 x 64.
#include "mq_device.hpp"
#include "mq_launch.hpp"

namespace mq {
namespace {

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDS_STRIDE = 40;  // halves per LDS row: 32 + 8 padding (conflict-free 16B reads)
constexpr int kThreads = 256;

struct TiledKArgs {
  const _Float16* A; int64_t lda;
  const unsigned char* W; int64_t ldw;
  const _Float16* scales; const _Float16* zeros;
  EpiArgs ep;
  _Float16* C; int64_t ldc;
  int M, N, K, g, G, F, gshift;
};

template <int FMT>
struct Stage {
  u4 a0, a1;    // 16 fp16 of A (row r, k half h)
  u4 w;         // int4: 2 dwords used (.x,.y); int8: 4 dwords
  _Float16 s, z;
};

template <int FMT, int EPI>
__global__ __launch_bounds__(kThreads, 2) void tiled_kernel(TiledKArgs p) {
  __shared__ __align__(16) _Float16 lds[2][2][BM * LDS_STRIDE];  // [buf][A/B][row*stride]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int m0 = blockIdx.y * BM;
  const int nb = blockIdx.x;

  // loader mapping: row r = tid/2, k half h = tid&1 (16 k values)
  const int lr = tid >> 1, lh = tid & 1;
  const int am = m0 + lr;
  const bool a_ok = am < p.M;
  const _Float16* arow = p.A + (int64_t)(a_ok ? am : 0) * p.lda + 16 * lh;
  int wn_row;
  bool w_ok;
  if (EPI == EPI_SWIGLU) {
    int j = nb * 64 + (lr & 63);
    w_ok = j < p.F;
    wn_row = (lr >= 64) ? p.F + j : j;
  } else {
    wn_row = nb * BN + lr;
    w_ok = wn_row < p.N;
  }
  const unsigned char* wrow = p.W + (int64_t)(w_ok ? wn_row : 0) * p.ldw;
  const int64_t srow = (int64_t)(w_ok ? wn_row : 0) * p.G;

  auto load = [&](int kt, Stage<FMT>& st) {
    const int k = kt * BK;
    st.a0 = (u4){0u, 0u, 0u, 0u};
    st.a1 = st.a0;
    st.w = st.a0;
    st.s = (_Float16)0.f;
    st.z = (_Float16)0.f;
    if (a_ok) {
      st.a0 = *(const u4*)(arow + k);
      st.a1 = *(const u4*)(arow + k + 8);
    }
    if (w_ok) {
      if (FMT == FMT_INT4) {
        const uint32_t* src = (const uint32_t*)(wrow + k / 2 + 8 * lh);
        st.w.x = __builtin_nontemporal_load(src);
        st.w.y = __builtin_nontemporal_load(src + 1);
      } else {
        st.w = __builtin_nontemporal_load((const u4*)(wrow + k + 16 * lh));
      }
      int gi = p.gshift >= 0 ? (k >> p.gshift) : (p.G == 1 ? 0 : k / p.g);
      st.s = p.scales[srow + gi];
      if (p.zeros) st.z = p.zeros[srow + gi];
    }
  };

  auto store = [&](int buf, const Stage<FMT>& st) {
    _Float16* as = &lds[buf][0][lr * LDS_STRIDE + 16 * lh];
    _Float16* bs = &lds[buf][1][lr * LDS_STRIDE + 16 * lh];
    u4 a0 = st.a0, a1 = st.a1;
    if (FMT == FMT_INT4) { a0 = perm8_int4(a0); a1 = perm8_int4(a1); }
    *(u4*)as = a0;
    *(u4*)(as + 8) = a1;
    // (built from the bits: a vector literal of two halves went through scratch memory)
    const uint32_t su = __builtin_bit_cast(uint16_t, st.s), zu = __builtin_bit_cast(uint16_t, st.z);
    const h2 s2 = as_h2(su | (su << 16)), z2 = as_h2(zu | (zu << 16));
    if (FMT == FMT_INT4) {
      *(h8*)bs = dq_int4_dword_perm(st.w.x, s2, z2);
      *(h8*)(bs + 8) = dq_int4_dword_perm(st.w.y, s2, z2);
    } else {
      h2 q0, q1, q2, q3, q4, q5, q6, q7;
      dq_int8_dword(st.w.x, s2, z2, q0, q1);
      dq_int8_dword(st.w.y, s2, z2, q2, q3);
      dq_int8_dword(st.w.z, s2, z2, q4, q5);
      dq_int8_dword(st.w.w, s2, z2, q6, q7);
      h8 b0, b1;
      b0.s01 = q0; b0.s23 = q1; b0.s45 = q2; b0.s67 = q3;
      b1.s01 = q4; b1.s23 = q5; b1.s45 = q6; b1.s67 = q7;
      *(h8*)bs = b0;
      *(h8*)(bs + 8) = b1;
    }
  };

  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

  const int KT = p.K / BK;
  Stage<FMT> st;
  load(0, st);
  store(0, st);
  __syncthreads();
  const int rl = lane & 15, kg = 8 * (lane >> 4);
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load(kt + 1, st);
    const _Float16* as = lds[buf][0];
    const _Float16* bs = lds[buf][1];
    h8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *(const h8*)(as + (wm * 64 + 16 * i + rl) * LDS_STRIDE + kg);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = *(const h8*)(bs + (wn * 64 + 16 * j + rl) * LDS_STRIDE + kg);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(a[i], b[j], acc[i][j]);
    if (kt + 1 < KT) store(buf ^ 1, st);
    __syncthreads();
  }

  // ---- epilogue ----
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) mfma_result_fence(acc[i][j]);
  // Lane holds D[row = 16*i + 4*(lane>>4) + r][col = 16*j + (lane&15)] of the wave sub-tile.
  if (EPI == EPI_SWIGLU) {
    // up waves (wn == 1) hand half(up) to the gate waves through LDS
    _Float16* up = &lds[0][0][0];  // [128][64] fp16 = 16 KiB, fits in buffer 0
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            up[(wm * 64 + 16 * i + 4 * (lane >> 4) + r) * 64 + 16 * j + (lane & 15)] =
                (_Float16)acc[i][j][r];
    }
    __syncthreads();
    if (wn == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int rr = wm * 64 + 16 * i + 4 * (lane >> 4) + r;
            int cc = 16 * j + (lane & 15);
            int m = m0 + rr, col = nb * 64 + cc;
            if (m < p.M && col < p.F) {
              float gv = (float)(_Float16)acc[i][j][r];
              float uv = (float)up[rr * 64 + cc];
              p.C[(int64_t)m * p.ldc + col] = (_Float16)(silu_f32(gv) * uv);
            }
          }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int col = nb * BN + wn * 64 + 16 * j + (lane & 15);
        if (col >= p.N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int m = m0 + wm * 64 + 16 * i + 4 * (lane >> 4) + r;
          if (m < p.M) p.C[(int64_t)m * p.ldc + col] = (_Float16)epi_apply(acc[i][j][r], m, col, p.ep);
        }
      }
  }
}

template <int FMT>
hipError_t launch_fmt(const TiledKArgs& k, int epi, dim3 grid, hipStream_t s) {
  if (epi == EPI_SWIGLU)
    hipLaunchKernelGGL((tiled_kernel<FMT, EPI_SWIGLU>), grid, dim3(kThreads), 0, s, k);
  else
    hipLaunchKernelGGL((tiled_kernel<FMT, EPI_NONE>), grid, dim3(kThreads), 0, s, k);
  return hipGetLastError();
}

}  // namespace

bool tiled_supported(const LinearArgs& a) {
  if (a.fmt != FMT_INT4 && a.fmt != FMT_INT8) return false;
  if (a.K % BK != 0) return false;
  if (a.g % BK != 0) return false;  // one group per row per K step
  if (((uintptr_t)a.A & 15) || (a.lda & 7)) return false;
  if (((uintptr_t)a.W & 15) || (a.ldw & 15)) return false;
  if (a.epi == EPI_SWIGLU && a.F * 2 != a.N) return false;
  return true;
}

hipError_t tiled_launch(const LinearArgs& a, hipStream_t s) {
  TiledKArgs k{};
  k.A = (const _Float16*)a.A; k.lda = a.lda;
  k.W = (const unsigned char*)a.W; k.ldw = a.ldw;
  k.scales = (const _Float16*)a.scales; k.zeros = (const _Float16*)a.zeros;
  k.ep = a.epi_args();
  k.C = (_Float16*)a.C; k.ldc = a.ldc;
  k.M = a.M; k.N = a.N; k.K = a.K; k.g = a.g; k.G = a.G; k.F = a.F;
  k.gshift = -1;
  for (int b = 0; b < 31; ++b)
    if (a.g == (1 << b)) k.gshift = b;
  int ntiles = (a.epi == EPI_SWIGLU) ? (a.F + 63) / 64 : (a.N + BN - 1) / BN;
  dim3 grid(ntiles, (a.M + BM - 1) / BM);
  switch (a.fmt) {
    case FMT_INT4: return launch_fmt<FMT_INT4>(k, a.epi, grid, s);
    default: return launch_fmt<FMT_INT8>(k, a.epi, grid, s);
  }
}

}  // namespace mq
