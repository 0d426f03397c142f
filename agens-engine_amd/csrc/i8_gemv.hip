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
// per token and applied to all of the half-wave's rows (4 for one token, else 2).  A workgroup of 256 threads is 8
// half-waves.  The weight stream is
// the only large traffic: at m = 1 the kernel is bounded by HBM (1 byte per weight), from about m = 4 on by the
// VALU (one fma per weight and token).
#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {
namespace {

// rows per half-wave: 4 for one token (the activation chunk's conversion shared by more rows), 2 with more tokens
// (their accumulators take the registers)
template <int MT>
constexpr int rows_of() { return MT == 1 ? 4 : 2; }

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
// signed byte B of w as an exact float, one instruction: v_cvt_f32_i32 of the sign-extended byte (SDWA byte select).
// Written out because this toolchain turns (float) of a sign-extended byte into v_cvt_f32_u32 with the same
// sign-extending operand, which converts a negative byte as a large unsigned value.
template <int B>
__device__ __forceinline__ float i8_of(uint32_t w) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
  else if constexpr (B == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
  else if constexpr (B == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
  return r;
}

// the 16 weights of a chunk word by word as exact floats
__device__ __forceinline__ void chunk_f32(const uint4 q, float (&f)[16]) {
  const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[4 * i + 0] = i8_of<0>(wd[i]);
    f[4 * i + 1] = i8_of<1>(wd[i]);
    f[4 * i + 2] = i8_of<2>(wd[i]);
    f[4 * i + 3] = i8_of<3>(wd[i]);
  }
}

// XL: the activations (m * k bf16) staged in LDS by the workgroup, then read from there (one token, k * 2 <= 32 KB)
template <int MT, bool XL>
__global__ void __launch_bounds__(256) i8_gemv_kernel(const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
                                                      const float* __restrict__ scale, uint16_t* __restrict__ y, int m,
                                                      int n, int k, int ldy) {
  constexpr int kRows = rows_of<MT>();
  __shared__ __attribute__((aligned(16))) uint4 xs[XL ? 2048 : 1];
  if constexpr (XL) {
    const uint4* xg = reinterpret_cast<const uint4*>(x);
    for (int i = threadIdx.x; i < (m * k) >> 3; i += 256) xs[i] = xg[i];
    __syncthreads();
  }
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
  // the next chunk's weights are requested before this chunk is computed (two chunks in flight per row); the two
  // half-waves of a wave read different rows: per-lane addresses
  u32x4 nx[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
    nx[r] = l < chunks ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr[r] + (size_t)l * 16))
                       : u32x4{0u, 0u, 0u, 0u};
  for (int c = l; c < chunks; c += 32) {
    float qf[kRows][16];
    u32x4 cur[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) cur[r] = nx[r];
    if (c + 32 < chunks) {
#pragma unroll
      for (int r = 0; r < kRows; ++r)
        nx[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr[r] + (size_t)(c + 32) * 16));
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) chunk_f32(make_uint4(cur[r][0], cur[r][1], cur[r][2], cur[r][3]), qf[r]);
    // tokens: every j < MT unrolled (a guard, not a loop exit, so that the accumulators stay in registers)
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j < m) {
        const uint4* xr = (XL ? xs : reinterpret_cast<const uint4*>(x)) + (((size_t)j * k) >> 3) + 2 * c;
        const uint4 a = xr[0], b = xr[1];
        const uint32_t xw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float xf[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) xf[2 * i] = bf_lo(xw[i]), xf[2 * i + 1] = bf_hi(xw[i]);
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
          float s = 0.f;
#pragma unroll
          for (int e = 0; e < 16; ++e) s = __builtin_fmaf(xf[e], qf[r][e], s);
          acc[r][j] += s;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int o = o0 + r;
    const float sc = o < n ? scale[o] : 0.f;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j < m) {
        float v = acc[r][j];
#pragma unroll
        for (int d = 16; d > 0; d >>= 1) v += __shfl_xor(v, d, 32);
        if (l == 0 && o < n) y[(size_t)j * ldy + o] = f2bf(v * sc);
      }
    }
  }
}

}  // namespace
}  // namespace agq

extern "C" int ak_i8_gemv(const void* x, const void* w, const void* scale, void* y, int m, int n, int k, int ldy,
                          void* stream) {
  // the reference's checks (i8_gemv.cu:74), and null pointers / empty shapes
  if (!x || !w || !scale || !y || m < 1 || m > 16 || n < 1 || k < 16 || k % 16) return AK_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  auto W = static_cast<const int8_t*>(w);
  auto S = static_cast<const float*>(scale);
  auto Y = static_cast<uint16_t*>(y);
  auto wgs = [n](int rows) { return dim3((n + 8 * rows - 1) / (8 * rows)); };  // 8 half-waves per workgroup
  if (m == 1 && k <= 16384)
    hipLaunchKernelGGL((agq::i8_gemv_kernel<1, true>), wgs(agq::rows_of<1>()), dim3(256), 0, s, X, W, S, Y, m, n, k,
                       ldy);
  else if (m == 1)
    hipLaunchKernelGGL((agq::i8_gemv_kernel<1, false>), wgs(agq::rows_of<1>()), dim3(256), 0, s, X, W, S, Y, m, n, k,
                       ldy);
  else if (m <= 8)
    hipLaunchKernelGGL((agq::i8_gemv_kernel<8, false>), wgs(agq::rows_of<8>()), dim3(256), 0, s, X, W, S, Y, m, n, k,
                       ldy);
  else
    hipLaunchKernelGGL((agq::i8_gemv_kernel<16, false>), wgs(agq::rows_of<16>()), dim3(256), 0, s, X, W, S, Y, m, n,
                       k, ldy);
  return (int)hipGetLastError();
}
