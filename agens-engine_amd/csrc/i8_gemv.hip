// INT8-weight GEMV for the LM head (W8A16, one fp32 scale per output row), gfx950:
//   y[j][o] (row stride ldy) = bf16(scale[o] * sum_i x[j][i] * q[o][i]),  q int8 [n][k], 1 <= m <= 16, k % 16 == 0.
// Reference: ak_i8_gemv, kernels/src/i8_gemv.cu:28-88.  The reference's numerics are an fp32 order that does not
// depend on m, and this kernel keeps that order exactly, so its results are bit-identical to the reference's:
//   - 32 partial sums per (row, token), partial l over the 16-input chunks c = l, l + 32, l + 64, ... in that order;
//   - per chunk, s = 0 and then s = fma(x_e, q_e, s) for its inputs e = 0..15 in order, and partial += s;
//   - the 32 partials reduced by an xor butterfly (distance 16, 8, 4, 2, 1: v += v[l ^ d]); the result times the
//     row's scale, rounded to bf16 (nearest even).
// Layout on MI355X: a half-wave (32 lanes) plays the reference's warp for kRows rows at once (the lanes' chunk loads
// of a row are 512 contiguous bytes, one 16-byte non-temporal load per lane); the activations' chunk is loaded once
// per token and applied to all kRows rows.  A workgroup of 256 threads covers 8 * kRows rows.  The weight stream is
// the only large traffic: at m = 1 the kernel is bounded by HBM (1 byte per weight), from about m = 4 on by the
// VALU (one fma per weight and token).
#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {
namespace {

constexpr int kRows = 2;  // rows per half-wave

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
// signed byte b of w, exactly: (byte ^ 0x80) is q + 128 in [0, 255] (one unsigned byte conversion), minus 128.  Not
// (float) of a sign-extended byte: this toolchain turns that into v_cvt_f32_u32 with a sign-extending byte operand,
// which converts a negative byte as a large unsigned value.
__device__ __forceinline__ float i8_of(uint32_t w, int b) {
  return (float)(((w ^ 0x80808080u) >> (8 * b)) & 0xFFu) - 128.f;
}

// s = fma(x_e, q_e, s) over the 4 inputs of weight word w (x01: inputs 0, 1; x23: inputs 2, 3)
__device__ __forceinline__ float dot4(uint32_t w, uint32_t x01, uint32_t x23, float s) {
  s = __builtin_fmaf(bf_lo(x01), i8_of(w, 0), s);
  s = __builtin_fmaf(bf_hi(x01), i8_of(w, 1), s);
  s = __builtin_fmaf(bf_lo(x23), i8_of(w, 2), s);
  s = __builtin_fmaf(bf_hi(x23), i8_of(w, 3), s);
  return s;
}

template <int MT>
__global__ void __launch_bounds__(256) i8_gemv_kernel(const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
                                                      const float* __restrict__ scale, uint16_t* __restrict__ y, int m,
                                                      int n, int k, int ldy) {
  const int l = threadIdx.x & 31;                                          // the reference's lane
  const int hw = threadIdx.x >> 5;                                         // half-wave of the workgroup
  const int o0 = (blockIdx.x * (256 / 32) + hw) * kRows;                   // first row of this half-wave
  const int chunks = k >> 4;
  float acc[kRows][MT];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[r][j] = 0.f;
  // rows past n read row n - 1 (results not written)
  const int8_t* wr[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) wr[r] = w + (size_t)(o0 + r < n ? o0 + r : n - 1) * k;
  for (int c = l; c < chunks; c += 32) {
    uint4 q[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {  // the two half-waves of a wave read different rows: per-lane addresses
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr[r] + (size_t)c * 16));
      q[r] = make_uint4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j >= m) break;
      const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)j * k) + 2 * c;
      const uint4 a = xr[0], b = xr[1];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        float s = 0.f;
        s = dot4(q[r].x, a.x, a.y, s);
        s = dot4(q[r].y, a.z, a.w, s);
        s = dot4(q[r].z, b.x, b.y, s);
        s = dot4(q[r].w, b.z, b.w, s);
        acc[r][j] += s;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int o = o0 + r;
    const float sc = o < n ? scale[o] : 0.f;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j >= m) break;
      float v = acc[r][j];
#pragma unroll
      for (int d = 16; d > 0; d >>= 1) v += __shfl_xor(v, d, 32);
      if (l == 0 && o < n) y[(size_t)j * ldy + o] = f2bf(v * sc);
    }
  }
}

}  // namespace
}  // namespace agq

extern "C" int ak_i8_gemv(const void* x, const void* w, const void* scale, void* y, int m, int n, int k, int ldy,
                          void* stream) {
  // the reference's checks (i8_gemv.cu:74), and null pointers / empty shapes
  if (!x || !w || !scale || !y || m < 1 || m > 16 || n < 1 || k < 16 || k % 16) return AK_INVALID;
  const int wg = (n + 8 * agq::kRows - 1) / (8 * agq::kRows);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  auto W = static_cast<const int8_t*>(w);
  auto S = static_cast<const float*>(scale);
  auto Y = static_cast<uint16_t*>(y);
  if (m == 1)
    hipLaunchKernelGGL(agq::i8_gemv_kernel<1>, dim3(wg), dim3(256), 0, s, X, W, S, Y, m, n, k, ldy);
  else if (m <= 8)
    hipLaunchKernelGGL(agq::i8_gemv_kernel<8>, dim3(wg), dim3(256), 0, s, X, W, S, Y, m, n, k, ldy);
  else
    hipLaunchKernelGGL(agq::i8_gemv_kernel<16>, dim3(wg), dim3(256), 0, s, X, W, S, Y, m, n, k, ldy);
  return (int)hipGetLastError();
}
