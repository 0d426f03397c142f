// Batch-invariant bf16 GEMV for small m (speculative decoding: a verify of m tokens must give every token the bits a
// one-token step gives it), gfx950:
//   y[t][r] (row stride ldy) = bf16(sum_i x[t][i] * W[r][i] (+ bias[r])),  W bf16 [n][k] row-major, 1 <= m <= 128,
//   k % 32 == 0.
// Reference: ak_bf16_gemv_bi / _ld, kernels/src/bi_gemv.cu:270-356 (tensor-core MMA kernels whose per-token order is the
// same for every m).  The reference's bits come from its MMA instruction's internal accumulation, which no other
// hardware reproduces; this kernel keeps the reference's contract instead -- fp32 accumulation, the bias added in fp32
// before the one bf16 rounding, and an order that does not depend on m:
//   - a workgroup owns 16 rows; its 8 waves take the 64-input k-steps s = w, w + 8, w + 16, ... (wave w; four steps'
//     loads issued at a time), each step two
//     v_mfma_f32_16x16x32_bf16 (inputs [64 s, 64 s + 32) then [64 s + 32, 64 s + 64)) accumulating in fp32;
//   - the MFMA's A operand is 16 weight rows, its B operand 16 tokens: the columns of the result are independent, so a
//     token's sums do not depend on the other tokens; more than 16 tokens are more B tiles of the same steps;
//   - the 8 waves' partial sums are added in wave order (from wave 0), then the bias, then the bf16 rounding.
// Operand layout: lane l holds inputs 8 (l / 16) .. + 8 of row (A) / token (B) l % 16 of the 32-input slice (one 16-byte
// load each); any input-to-slot map gives the same sum as long as A and B use the same one.  D: lane l holds rows
// 4 (l / 16) + i, i < 4, of token l % 16.
#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kWaves = 8;

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4 v) {
  bf16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// TT token tiles of 16 per launch (tokens [0, 16 TT) of x; m <= 16 TT)
template <int TT>
__global__ void __launch_bounds__(kWaves * 64) bi_gemv_kernel(const uint16_t* __restrict__ x, int m,
                                                              const uint16_t* __restrict__ w,
                                                              const uint16_t* __restrict__ bias,
                                                              uint16_t* __restrict__ y, int n, int k, long ldy) {
  __shared__ f32x4 red[kWaves][TT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = (int)blockIdx.x * 16 + (lane & 15);  // this lane's A row
  const int kq = 8 * (lane >> 4);                      // its inputs within a 32-input slice
  const bool rok = r < n;
  const uint16_t* wr = w + (size_t)(rok ? r : 0) * k + kq;
  f32x4 acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int steps = (k + 63) >> 6;
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  // KU of the wave's steps at a time: their weight loads (and with one token tile their activation loads) are issued
  // together, then their MFMAs in step order -- the same chain as one step at a time
  constexpr int KU = 4;
  for (int s0 = wave; s0 < steps; s0 += kWaves * KU) {
    uint4 a0[KU], a1[KU], b0[KU], b1[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      // unconditional 16-byte loads at clamped (always valid) offsets, zeros selected afterwards: a conditional load
      // would be split into guarded dword loads
      const int s = s0 + u * kWaves, k0 = 64 * s;
      const bool in = s < steps, two = k0 + 32 < k;
      const int ka = in ? k0 : 0, kb = in && two ? k0 + 32 : 0;
      const u32x4 va = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + ka));
      const u32x4 vb = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + kb));
      a0[u] = rok && in ? make_uint4(va[0], va[1], va[2], va[3]) : z;
      a1[u] = rok && in && two ? make_uint4(vb[0], vb[1], vb[2], vb[3]) : z;
      if constexpr (TT == 1) {
        const int tok = lane & 15;
        const uint16_t* xr = x + (size_t)(tok < m ? tok : 0) * k + kq;
        const uint4 xa = *reinterpret_cast<const uint4*>(xr + ka), xb = *reinterpret_cast<const uint4*>(xr + kb);
        b0[u] = tok < m && in ? xa : z;
        b1[u] = tok < m && in && two ? xb : z;
      }
    }
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int s = s0 + u * kWaves, k0 = 64 * s;
      if (s >= steps) break;
      const bool two = k0 + 32 < k;  // k % 32 == 0: the step's second slice exists unless k ends at k0 + 32
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        uint4 xb0 = b0[u], xb1 = b1[u];
        if constexpr (TT > 1) {
          const int tok = 16 * t + (lane & 15);
          const bool tk = tok < m;
          const uint16_t* xr = x + (size_t)(tk ? tok : 0) * k + kq + k0;
          const uint4 xa = *reinterpret_cast<const uint4*>(xr), xb = *reinterpret_cast<const uint4*>(xr + (two ? 32 : 0));
          xb0 = tk ? xa : z;
          xb1 = tk && two ? xb : z;
        }
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0[u]), as_bf16x8(xb0), acc[t], 0, 0, 0);
        if (two) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1[u]), as_bf16x8(xb1), acc[t], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  // thread (tile t, lane) of the first TT waves adds the waves' partials in wave order, then the bias, and writes its
  // 4 rows of token 16 t + lane % 16
  if (wave < TT) {
    const int t = wave;
    f32x4 v = red[0][t][lane];
#pragma unroll
    for (int ww = 1; ww < kWaves; ++ww) v += red[ww][t][lane];
    const int tok = 16 * t + (lane & 15);
    if (tok < m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (int)blockIdx.x * 16 + 4 * (lane >> 4) + i;
        if (row < n) {
          const float b = bias ? __uint_as_float((uint32_t)bias[row] << 16) : 0.f;
          y[(size_t)tok * ldy + row] = f2bf(bias ? v[i] + b : v[i]);
        }
      }
    }
  }
}

}  // namespace
}  // namespace agq

extern "C" int ak_bf16_gemv_bi_ld(const void* x, const void* w, const void* bias, void* y, int m, int n, int k, long ldy,
                                  void* stream) {
  // the reference's checks (bi_gemv.cu:276), null pointers / empty shapes, and a row stride below n (token rows would
  // overlap)
  if (!x || !w || !y || m < 1 || m > 128 || n < 1 || k < 32 || k % 32 != 0 || ldy < n) return AK_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  auto W = static_cast<const uint16_t*>(w);
  auto B = static_cast<const uint16_t*>(bias);
  auto Y = static_cast<uint16_t*>(y);
  const dim3 grid((n + 15) / 16), block(agq::kWaves * 64);
  const int tt = (m + 15) / 16;
  switch (tt) {
    case 1: hipLaunchKernelGGL(agq::bi_gemv_kernel<1>, grid, block, 0, s, X, m, W, B, Y, n, k, ldy); break;
    case 2: hipLaunchKernelGGL(agq::bi_gemv_kernel<2>, grid, block, 0, s, X, m, W, B, Y, n, k, ldy); break;
    case 3:
    case 4: hipLaunchKernelGGL(agq::bi_gemv_kernel<4>, grid, block, 0, s, X, m, W, B, Y, n, k, ldy); break;
    default: hipLaunchKernelGGL(agq::bi_gemv_kernel<8>, grid, block, 0, s, X, m, W, B, Y, n, k, ldy); break;
  }
  return (int)hipGetLastError();
}

extern "C" int ak_bf16_gemv_bi(const void* x, const void* w, const void* bias, void* y, int m, int n, int k,
                               void* stream) {
  return ak_bf16_gemv_bi_ld(x, w, bias, y, m, n, k, n, stream);
}
