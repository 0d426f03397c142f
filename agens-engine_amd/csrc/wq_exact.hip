// The reference's "exact" fp32 GEMV numerics on gfx950 (selected by ak_w4_set_mma(0) / AGENS_W4_EXACT=1, and for
// bf16w = 1).  Output bits equal the reference's w4_gemv_kt_kernel / w4_gemv_kt_batched_kernel / w4g128_gemv_kernel
// (kernels/src/w4_gemv.cu:112-127, :129-190, :279-349, :367-437):
//   per output row, "lane" l of 32 owns chunk 32t + l of every tile t; per chunk the 32-input dot product is four
//   8-term fma chains (x as fp32, q = nibble - 8 exact) added left to right, then acc = fma(d, scale, acc)
//   (bf16w: weights first rounded to bf16(q * scale), acc += d); then a xor butterfly over the 32 lanes (16, 8, 4,
//   2, 1) and one bf16 rounding.
// On wave64 each half-wave (32 lanes) plays the role of one such row unit; the butterfly stays inside the half.
#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {

int num_cus();

namespace {

constexpr int kThreads = 256;  // 4 waves = 8 row units per block

__device__ __forceinline__ uint32_t spread2(uint32_t v) {
  v &= 0xFFFFu;
  v = (v ^ (v << 8)) & 0x00FF00FFu;
  v = (v ^ (v << 4)) & 0x0F0F0F0Fu;
  return (v ^ (v << 2)) & 0x33333333u;
}
__device__ __forceinline__ uint32_t spread1(uint32_t v) {
  v &= 0xFFu;
  v = (v ^ (v << 12)) & 0x000F000Fu;
  v = (v ^ (v << 6)) & 0x03030303u;
  return (v ^ (v << 3)) & 0x11111111u;
}

// a lane chunk's raw KT words (W4: the nibble chunk; W3: two-bit plane words + third-bit plane word; W2: plane words),
// and their decoding into W4 nibble words (nibble = q + 8) -- separate, so that a chunk can be requested a tile ahead
// and decoded when it is used
struct RawChunk {
  uint4 w;  // W4: the chunk; W2 / W3: .x .y the two-bit plane, .z the third-bit plane (W3)
};
template <int BITS>
__device__ __forceinline__ RawChunk load_raw_chunk(const void* __restrict__ wt, size_t rec, int c) {
  RawChunk r;
  if (BITS == 4) {
    r.w = ld_stream(reinterpret_cast<const uint4*>(wt) + rec * 32 + c);
  } else {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(wt) + rec * (32 * BITS);
    const uint2 lo = reinterpret_cast<const uint2*>(p)[c];
    r.w = make_uint4(lo.x, lo.y, BITS == 3 ? p[64 + c] : 0u, 0u);
  }
  return r;
}
template <int BITS>
__device__ __forceinline__ uint4 decode_chunk(const RawChunk& r) {
  if (BITS == 4) return r.w;
  const uint32_t lx = r.w.x, ly = r.w.y;
  if (BITS == 2)
    return make_uint4(spread2(lx) + 0x66666666u, spread2(lx >> 16) + 0x66666666u, spread2(ly) + 0x66666666u,
                      spread2(ly >> 16) + 0x66666666u);
  const uint32_t h = r.w.z;
  return make_uint4((spread2(lx) | (spread1(h) << 2)) + 0x44444444u,
                    (spread2(lx >> 16) | (spread1(h >> 8) << 2)) + 0x44444444u,
                    (spread2(ly) | (spread1(h >> 16) << 2)) + 0x44444444u,
                    (spread2(ly >> 16) | (spread1(h >> 24) << 2)) + 0x44444444u);
}

// nibble i of w as an exact fp32 q = nibble - 8, from w8 = w ^ 0x88888888 (nibble ^ 8 is q as a 4-bit two's
// complement field): a sign-extending field extract (a shift pair) and one conversion.  Not __builtin_amdgcn_sbfe:
// this toolchain converts its result as if it were unsigned (v_cvt_f32_u32), which is wrong for the negative codes.
__device__ __forceinline__ float nibq(uint32_t w8, int i) { return (float)((int)(w8 << (28 - 4 * i)) >> 28); }

// the 32 inputs of a lane chunk as fp32 (XF: already fp32 in LDS; else 16 words of bf16 pairs)
struct ChunkX {
  float v[32];
};
__device__ __forceinline__ void chunk_x_bf16(const uint32_t* xp, ChunkX& cx) {
#pragma unroll
  for (int p = 0; p < 16; ++p) cx.v[2 * p] = __uint_as_float(xp[p] << 16), cx.v[2 * p + 1] = __uint_as_float(xp[p] & 0xFFFF0000u);
}

// dot of one nibble word (8 inputs) with its 8 inputs: the fixed fma chain
template <bool BW>
__device__ __forceinline__ float dot8(uint32_t w, const float* xv, float sc) {
  const uint32_t w8 = w ^ 0x88888888u;
  float s = 0.f;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float a = nibq(w8, 2 * p), b = nibq(w8, 2 * p + 1);
    if (BW) a = bf2f(f2bf(a * sc)), b = bf2f(f2bf(b * sc));
    s = fmaf(xv[2 * p], a, s);
    s = fmaf(xv[2 * p + 1], b, s);
  }
  return s;
}

template <bool BW>
__device__ __forceinline__ float chunk_step(const uint4& w, const ChunkX& cx, float sc, float acc) {
  const float d = dot8<BW>(w.x, cx.v, sc) + dot8<BW>(w.y, cx.v + 8, sc) + dot8<BW>(w.z, cx.v + 16, sc) +
                  dot8<BW>(w.w, cx.v + 24, sc);
  return BW ? acc + d : fmaf(d, sc, acc);
}

__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// KT layout, m tokens (MT = 1: x staged in LDS chunk-transposed, XF: as fp32, 4 inputs per 16-byte read; MT > 1: up
// to MT tokens, x read from global).
template <int BITS, int G, bool BW, int MT, bool XF = false>
__global__ void __launch_bounds__(kThreads) exact_kernel(const uint16_t* __restrict__ x, int m, const Segs segs,
                                                         int k) {
  extern __shared__ uint32_t xs[];
  constexpr int SPT = 1024 / G, CPG = G / 32;
  const int kp = kpad(k), chunks = kp >> 5, tiles = kp >> 10, kc = k >> 5;
  if (MT == 1 && XF) {  // [quad q of 4 inputs][chunk c] float4: chunk c's inputs 4q .. 4q + 3
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
    float4* const x4 = reinterpret_cast<float4*>(xs);
    for (int i = threadIdx.x; i < (kp >> 2); i += kThreads) {
      const uint32_t a = 2 * i < (k >> 1) ? xw[2 * i] : 0u, b = 2 * i + 1 < (k >> 1) ? xw[2 * i + 1] : 0u;
      x4[(i & 7) * chunks + (i >> 3)] = make_float4(__uint_as_float(a << 16), __uint_as_float(a & 0xFFFF0000u),
                                                    __uint_as_float(b << 16), __uint_as_float(b & 0xFFFF0000u));
    }
    __syncthreads();
  } else if (MT == 1) {
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
    for (int i = threadIdx.x; i < (kp >> 1); i += kThreads) xs[(i & 15) * chunks + (i >> 4)] = i < (k >> 1) ? xw[i] : 0u;
    __syncthreads();
  }
  const int lane = threadIdx.x & 31;
  const int unit0 = blockIdx.x * (kThreads / 32) + (threadIdx.x >> 5), units = gridDim.x * (kThreads / 32);
  const int rows = segs.end[segs.nseg - 1];
  for (int grow = unit0; grow < rows; grow += units) {
    const int sg = seg_of(segs, grow);
    const int o = grow - (sg ? segs.end[sg - 1] : 0), n = segs.n[sg];
    const void* wt = segs.wt[sg];
    const uint16_t* st = segs.st[sg];
    float acc[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[j] = 0.f;
    // the next tile's chunk and scale are requested before this tile is computed
    RawChunk wn = load_raw_chunk<BITS>(wt, o, lane);
    uint16_t sn = st[(size_t)o * SPT + lane / CPG];
    for (int t = 0; t < tiles; ++t) {
      const RawChunk wr = wn;
      const uint16_t sr = sn;
      if (t + 1 < tiles) {
        const size_t rn = (size_t)(t + 1) * n + o;
        wn = load_raw_chunk<BITS>(wt, rn, lane);
        sn = st[rn * SPT + lane / CPG];
      }
      const uint4 w = decode_chunk<BITS>(wr);
      const float sc = bf2f(sr);
      const int c = t * 32 + lane;
      if (MT == 1 && XF) {
        ChunkX cx;
        const float4* x4 = reinterpret_cast<const float4*>(xs);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float4 f = x4[q * chunks + c];
          cx.v[4 * q] = f.x, cx.v[4 * q + 1] = f.y, cx.v[4 * q + 2] = f.z, cx.v[4 * q + 3] = f.w;
        }
        acc[0] = chunk_step<BW>(w, cx, sc, acc[0]);
      } else if (MT == 1) {
        uint32_t xp[16];
#pragma unroll
        for (int p = 0; p < 16; ++p) xp[p] = xs[p * chunks + c];
        ChunkX cx;
        chunk_x_bf16(xp, cx);
        acc[0] = chunk_step<BW>(w, cx, sc, acc[0]);
      } else {
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          if (j >= m) break;
          uint32_t xp[16];
          if (c < kc) {
            const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)j * k + (size_t)c * 32);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint4 v = xr[q];
              xp[4 * q] = v.x, xp[4 * q + 1] = v.y, xp[4 * q + 2] = v.z, xp[4 * q + 3] = v.w;
            }
          } else {
#pragma unroll
            for (int p = 0; p < 16; ++p) xp[p] = 0u;
          }
          ChunkX cx;
          chunk_x_bf16(xp, cx);
          acc[j] = chunk_step<BW>(w, cx, sc, acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j >= m) break;
      const float v = half_wave_sum(acc[j]);
      if (lane == 0) segs.y[sg][(size_t)j * segs.ldy[sg] + o] = f2bf(v);
    }
  }
}

// int4 container (CT) layout, g128, m = 1 (the reference's legacy kernel, w4_gemv.cu:129-190): lane l walks chunks
// l, l + 32, ... of the row, exactly the KT lane order, so the bits equal the KT exact path.
__global__ void __launch_bounds__(kThreads) exact_ct_kernel(const uint16_t* __restrict__ x, const uint4* __restrict__ packed,
                                                            const uint16_t* __restrict__ scales, uint16_t* __restrict__ y,
                                                            int n, int k) {
  extern __shared__ uint32_t xs[];
  const int chunks = k >> 5, groups = k >> 7;
  const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);
  for (int i = threadIdx.x; i < (k >> 1); i += kThreads) xs[(i & 15) * chunks + (i >> 4)] = xw[i];
  __syncthreads();
  const int lane = threadIdx.x & 31;
  const int unit0 = blockIdx.x * (kThreads / 32) + (threadIdx.x >> 5), units = gridDim.x * (kThreads / 32);
  for (int o = unit0; o < n; o += units) {
    float acc = 0.f;
    for (int c = lane; c < chunks; c += 32) {
      const uint4 w = ld_stream(packed + (size_t)o * chunks + c);
      const float sc = bf2f(scales[(size_t)o * groups + (c >> 2)]);
      uint32_t xp[16];
#pragma unroll
      for (int p = 0; p < 16; ++p) xp[p] = xs[p * chunks + c];
      ChunkX cx;
      chunk_x_bf16(xp, cx);
      acc = chunk_step<false>(w, cx, sc, acc);
    }
    const float v = half_wave_sum(acc);
    if (lane == 0) y[o] = f2bf(v);
  }
}

template <int BITS, int G, bool BW, int MT>
int launch_exact(const void* x, int m, const Segs& g, int k, hipStream_t s) {
  // one token: x as fp32 in LDS while that leaves room for several workgroups per CU (k <= 8192), else as bf16
  const bool xf = MT == 1 && kpad(k) <= 8192;
  const size_t smem = MT == 1 ? (size_t)kpad(k) * (xf ? 4 : 2) : 0;
  const int rows = g.end[g.nseg - 1];
  const int want = (rows + kThreads / 32 - 1) / (kThreads / 32), cap = num_cus() * 8;
  if (xf)
    hipLaunchKernelGGL((exact_kernel<BITS, G, BW, MT, true>), dim3(want < cap ? want : cap), dim3(kThreads), smem, s,
                       static_cast<const uint16_t*>(x), m, g, k);
  else
    hipLaunchKernelGGL((exact_kernel<BITS, G, BW, MT>), dim3(want < cap ? want : cap), dim3(kThreads), smem, s,
                       static_cast<const uint16_t*>(x), m, g, k);
  return (int)hipGetLastError();
}

template <int BITS, int G, bool BW>
int exact_m(const void* x, int m, const Segs& g, int k, hipStream_t s) {
  if (m == 1) return launch_exact<BITS, G, BW, 1>(x, m, g, k, s);
  if (m <= 4) return launch_exact<BITS, G, BW, 4>(x, m, g, k, s);
  if (m <= 8) return launch_exact<BITS, G, BW, 8>(x, m, g, k, s);
  return launch_exact<BITS, G, BW, 16>(x, m, g, k, s);
}

template <int BITS>
int exact_bits(const void* x, int m, const Segs& g, int k, int group, int bf16w, hipStream_t s) {
  if (group == 64) return bf16w ? exact_m<BITS, 64, true>(x, m, g, k, s) : exact_m<BITS, 64, false>(x, m, g, k, s);
  return bf16w ? exact_m<BITS, 128, true>(x, m, g, k, s) : exact_m<BITS, 128, false>(x, m, g, k, s);
}

}  // namespace

// 1 <= m <= 16; segments padded with pad = 1 (Segs.end = cumulative n)
int exact_gemv(int bits, const void* x, int m, const Segs& g, int k, int group, int bf16w, hipStream_t s) {
  switch (bits) {
    case 4: return exact_bits<4>(x, m, g, k, group, bf16w, s);
    case 3: return exact_bits<3>(x, m, g, k, group, bf16w, s);
    case 2: return exact_bits<2>(x, m, g, k, group, bf16w, s);
    default: return AK_INVALID;
  }
}

int exact_ct_gemv(const void* x, const int32_t* packed, const void* scales, void* y, int n, int k, hipStream_t s) {
  const int want = (n + kThreads / 32 - 1) / (kThreads / 32), cap = num_cus() * 8;
  hipLaunchKernelGGL(exact_ct_kernel, dim3(want < cap ? want : cap), dim3(kThreads), (size_t)k * 2, s,
                     static_cast<const uint16_t*>(x), reinterpret_cast<const uint4*>(packed),
                     static_cast<const uint16_t*>(scales), static_cast<uint16_t*>(y), n, k);
  return (int)hipGetLastError();
}

}  // namespace agq
