// Prefill GEMM straight from the KT weights, gfx950: y[t][o] (row stride ldy) = bf16(sum_i x[t][i] * w[o][i]) with
// w[o][i] = bf16_rn(q * scale) -- the values ak_wq_dequant_kt_rows writes, bit for bit -- and fp32 accumulation.
//
// The reference's prefill route (kernels/m1/m1_model.cu:1876-1897) dequantizes a tile of output rows into a bf16
// scratch (2 bytes per weight written, then read again) and runs a library GEMM (ak_bf16_linear_f32reduce_ld,
// kernels/src/bf16_linear.cu:68-92).  Here the KT records are read once per token tile, expanded to bf16 in registers
// and written to LDS, and v_mfma_f32_16x16x32_bf16 consumes them there: no dequantized copy, no second pass over the
// weights (narrow linears split k across workgroups, with fp32 partials in the stream's split-K scratch).
//
// Two tilings, one kernel template (wq_gemm_kernel<BITS, G, R, T, RING, XR, XM, DMA>); k is walked in 64-input slabs.
//   - 128 x 128 (R = T = 128; 256 threads, 4 waves, two workgroups per CU), where few tiles exist (narrow linears):
//     thread (row tid / 2, half tid % 2) loads its lane chunk of the slab from the row's KT record (W4 16 B, W3
//     8 + 4 B, W2 8 B) and the group's scale, RING - 1 slabs ahead in a ring of registers; the inputs are 1024 16-byte
//     chunks per slab, 8 consecutive threads reading one token's 128 bytes, XR - 1 slabs ahead; both are written to
//     two LDS stages (16 KB weights, dequantized, + 16 KB inputs).  Grid: row tile major with the token tiles of a row
//     tile 8 workgroups apart (same XCD: workgroup i runs on XCD i % 8), sharing the row tile's weights in that L2.
//   - 256 x 256 (R = T = 256; 512 threads, 8 waves, one workgroup per CU), where the tiles fill the GPU (wide linears,
//     or from 2048 tokens): each weight is dequantized once per 256 tokens.  The tokens go straight from the buffer
//     into LDS (buffer loads into LDS, two stages of 32 KB, one slab ahead; no registers), the weights through a
//     register ring (W4 / W2 3 slabs ahead, W3 1) into two 32 KB stages; the next slab's dequantization is
//     interleaved with this slab's MFMAs (after each 16 MFMAs one of its four words; one MFMA, three VALU instructions
//     alternating), since the two waves of a SIMD leave the slab's barrier together.  Grid: the tiles in token-major order cut into 8
//     contiguous runs, XCD x taking run x, so that each XCD works on one or two token tiles (256 tokens x k inputs)
//     that stay in its L2 while the weights stream.
// Common: raw buffer loads with a per-lane offset fixed for the kernel and a scalar per-slab offset keep address
// arithmetic off the vector unit; no load sits under a branch (the compiler's wait counts stay exact).  LDS rows /
// tokens of 64 bf16 (128 B): the 16-byte chunk q of row r sits at slot q ^ ((r >> 1) & 7), so the 16 rows of one MFMA
// operand read hit 16 distinct 16-byte bank slots.  Wave tiles of 64 rows x 64 (128 x 128) or 128 (256 x 256)
// tokens, 16 x 16 MFMA tiles, two 32-input slices per slab; lane l reads 8 inputs 8 (l / 16) .. of its slice for row /
// token l % 16 (the same input-to-slot map for weights and tokens, which is all an MFMA needs).
// The accumulation order is this kernel's own (fp32 MFMA sums over 32 inputs, slabs in order): results agree with the
// reference's cuBLAS route and with the oracle's dequantized weights times x in fp64 within fp32-accumulation error.
#include <algorithm>
#include <type_traits>

#include "agens_kernels.h"
#include "wq_common.h"



namespace agq {
void* stream_scratch(hipStream_t s, size_t bytes);

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// slabs of 64 inputs (one row / token of a slab: 128 B in LDS), two LDS stages
constexpr int kSlab = 64, kRowBytes = kSlab * 2, kStages = 2;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, dword 3 (CDNA)

// f(integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>());
    static_for<B + 1, E>(f);
  }
}

__device__ __forceinline__ int swz(int r, int q) { return r * kRowBytes + ((q ^ ((r >> 1) & 7)) << 4); }

// the raw bits of one lane chunk (32 inputs) of a KT record and the scale of its group
template <int BITS>
struct ChunkRaw {
  u32x4 w;  // W4: the chunk; W3: lo words in 0, 1 and the third-bit word in 2; W2: lo words in 0, 1
  uint32_t s;
};

// 16 bytes per lane from a buffer straight into LDS: lane l writes dst + 16 l (dst the same for the whole wave)
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* dst, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

// Morton spreading of 2-bit / 1-bit fields into nibbles (as the repack's inverse)
__device__ __forceinline__ uint32_t spread2(uint32_t v) {
  v &= 0xFFFFu;
  v = (v ^ (v << 8)) & 0x00FF00FFu;
  v = (v ^ (v << 4)) & 0x0F0F0F0Fu;
  v = (v ^ (v << 2)) & 0x33333333u;
  return v;
}
__device__ __forceinline__ uint32_t spread1(uint32_t v) {
  v &= 0xFFu;
  v = (v ^ (v << 12)) & 0x000F000Fu;
  v = (v ^ (v << 6)) & 0x03030303u;
  v = (v ^ (v << 3)) & 0x11111111u;
  return v;
}

// the chunk as 4 words of 8 stored codes n (nibble i of word u = input 8 u + i) and the code offset: q = n - OFF
template <int BITS>
__device__ __forceinline__ void chunk_codes(const ChunkRaw<BITS>& d, uint32_t (&n)[4]) {
  if constexpr (BITS == 4) {
    n[0] = d.w[0], n[1] = d.w[1], n[2] = d.w[2], n[3] = d.w[3];
  } else if constexpr (BITS == 2) {
    n[0] = spread2(d.w[0]), n[1] = spread2(d.w[0] >> 16), n[2] = spread2(d.w[1]), n[3] = spread2(d.w[1] >> 16);
  } else {
    n[0] = spread2(d.w[0]) | (spread1(d.w[2]) << 2), n[1] = spread2(d.w[0] >> 16) | (spread1(d.w[2] >> 8) << 2);
    n[2] = spread2(d.w[1]) | (spread1(d.w[2] >> 16) << 2), n[3] = spread2(d.w[1] >> 16) | (spread1(d.w[2] >> 24) << 2);
  }
}

// 8 codes (one word) -> 8 bf16 bf16_rn((n - OFF) * s): the product is exact in fp32 (an fma of two exact terms), the
// conversion rounds to nearest even
template <int OFF>
__device__ __forceinline__ u32x4 dequant8(uint32_t w, float s) {
  const uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;  // codes of inputs 2b and 2b + 1 in byte b
  const float m = -(float)OFF * s;
  uint32_t o[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float lo = fmaf((float)((ev >> (8 * b)) & 0xFFu), s, m);
    const float hi = fmaf((float)((od >> (8 * b)) & 0xFFu), s, m);
    const bf16x2 p = {(__bf16)lo, (__bf16)hi};
    o[b] = __builtin_bit_cast(uint32_t, p);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// W2 / W3 without the nibble spread: the 2-bit codes of 16 inputs (one low word of the chunk, input i at bits 2i) as
// four words of byte codes, word p holding inputs 4 j + p in byte j (W3: the third bit, input i at bit i of the high
// half-word, merged at bit 2 of each byte through one 1-to-2 bit spread)
struct HalfCodes {
  uint32_t p0, p1, p2, p3;
};
template <int BITS>
__device__ __forceinline__ HalfCodes half_codes(const ChunkRaw<BITS>& d, int h) {
  const uint32_t L = d.w[h];
  HalfCodes c = {L & 0x03030303u, (L >> 2) & 0x03030303u, (L >> 4) & 0x03030303u, (L >> 6) & 0x03030303u};
  if constexpr (BITS == 3) {
    uint32_t v = (d.w[2] >> (16 * h)) & 0xFFFFu;  // third bits of inputs 16 h .. 16 h + 15; input i -> bit 2 i:
    v = (v | (v << 8)) & 0x00FF00FFu;
    v = (v | (v << 4)) & 0x0F0F0F0Fu;
    v = (v | (v << 2)) & 0x33333333u;
    v = (v | (v << 1)) & 0x55555555u;  // input 4 j + p at bit 8 j + 2 p
    c.p0 |= (v << 2) & 0x04040404u;
    c.p1 |= v & 0x04040404u;
    c.p2 |= (v >> 2) & 0x04040404u;
    c.p3 |= (v >> 4) & 0x04040404u;
  }
  return c;
}
// inputs 8 sub .. 8 sub + 7 of the half as 4 dwords of bf16 pairs bf16_rn((n - OFF) s) (as dequant8)
template <int OFF>
__device__ __forceinline__ u32x4 dequant_half(const HalfCodes& c, float s, int sub) {
  const float m = -(float)OFF * s;
  uint32_t o[4];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int sh = 8 * (2 * sub + jj);
    const bf16x2 ab = {(__bf16)fmaf((float)((c.p0 >> sh) & 0xFFu), s, m), (__bf16)fmaf((float)((c.p1 >> sh) & 0xFFu), s, m)};
    const bf16x2 cd = {(__bf16)fmaf((float)((c.p2 >> sh) & 0xFFu), s, m), (__bf16)fmaf((float)((c.p3 >> sh) & 0xFFu), s, m)};
    o[2 * jj] = __builtin_bit_cast(uint32_t, ab);
    o[2 * jj + 1] = __builtin_bit_cast(uint32_t, cd);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// R output rows x T tokens per workgroup (2 R threads: a thread pair per row), wave tiles of 64 rows x WT tokens,
// loads of the weights RING - 1 slabs ahead and of the tokens XR - 1 slabs ahead (RING a multiple of XR); XM: the
// XCD-contiguous tile order (below); DMA: the tokens are loaded straight into XR LDS stages of their own (buffer
// loads into LDS), not through registers
template <int BITS, int G, int R, int T, int RING, int XR, bool XM, bool DMA, bool SPLIT>
__global__ void __launch_bounds__(2 * R, R == 128 ? 2 : 1) wq_gemm_kernel(const uint16_t* __restrict__ x, int m,
                                                              const uint8_t* __restrict__ wt,
                                                              const uint16_t* __restrict__ st,
                                                              uint16_t* __restrict__ y, int n, int ldy, int k,
                                                              int nrow_tiles, int ntok_tiles, float* __restrict__ part) {
  constexpr int kRows = R, kToks = T, kThreads = 2 * R, kRing = RING;
  // LDS: DMA: two weight stages of R rows, then XR token stages of T tokens; else two stages of R rows + T tokens
  constexpr int kStage = DMA ? R * kRowBytes : (R + T) * kRowBytes, kXBase = DMA ? 2 * kStage : R * kRowBytes;
  constexpr int kXStage = DMA ? T * kRowBytes : kStage;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int OFF = BITS == 4 ? 8 : BITS == 3 ? 4 : 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // workgroup -> (row tile, token tile).  Workgroup b runs on XCD b % 8.  XM: the tiles in token-major order
  // (tile = token tile x row tiles + row tile) cut into 8 contiguous runs, XCD x taking run x, so that each XCD's
  // workgroups share one or two token tiles (T tokens x k inputs) through its L2 while the weights stream; else blocks
  // of 8 row tiles x all token tiles with the token tiles of a row tile 8 workgroups apart (same XCD: they share the
  // row tile's weights).
  const int b = blockIdx.x;
  int rt, tt;
  if constexpr (XM) {
    const int per = (nrow_tiles * ntok_tiles + 7) >> 3, tile = (b & 7) * per + (b >> 3);
    tt = tile / nrow_tiles, rt = tile - tt * nrow_tiles;
    if (tt >= ntok_tiles) return;
  } else {
    const int grp = b / (8 * ntok_tiles), in = b - grp * 8 * ntok_tiles;
    rt = grp * 8 + (in & 7), tt = in >> 3;
  }
  const int o0 = rt * kRows, t0 = tt * kToks;
  if (o0 >= n || t0 >= m) return;  // the last group of 8 row tiles may be partial

  // Per slab (64 inputs): thread (row lr, half lj) loads lane chunk 2 sl + lj of row lr's KT record (W4 16 B, W3
  // 8 + 4 B, W2 8 B) and its scale (rows past n load row n - 1: their results are not written); the inputs are 1024
  // 16-byte chunks (token c / 8, chunk c % 8), thread tid loading chunks tid + j * kThreads (8 consecutive threads read
  // one token's 128 bytes; tokens past m read token 0 and are written as zeros).  Loads are issued kRing - 1 slabs
  // ahead and every load is unconditional (a slab past the end loads the last one again, never used): loads under a
  // branch make the compiler's wait counts conservative at the join, which drains the pipeline.
  constexpr int XPT = kToks * 8 / kThreads;  // input chunks per thread and slab
  constexpr int REC = 128 * BITS, CB = BITS == 4 ? 16 : 8;  // record bytes; bytes of a lane chunk's (low) words
  const int lr = tid >> 1, lj = tid & 1;
  const int orow = o0 + lr < n ? o0 + lr : n - 1;
  // split-K (part != nullptr): workgroup (.., blockIdx.y) takes slabs [sb, sb + nslab) of the k range and writes its
  // fp32 tile to part[blockIdx.y][token][row] (row stride n); a second kernel adds the splits in order
  const int sb = SPLIT ? (int)((long long)blockIdx.y * (k / kSlab) / gridDim.y) : 0;
  const int nslab = SPLIT ? (int)((long long)(blockIdx.y + 1) * (k / kSlab) / gridDim.y) - sb : k / kSlab;
  // buffer loads: a per-lane offset fixed for the whole loop plus a per-slab scalar offset (no address arithmetic on
  // the vector unit in the loop); every buffer is below 2 GB (checked by the launcher)
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wt), (short)0, 0x7FFFFFFF,
                                                                      kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(st), (short)0, 0x7FFFFFFF,
                                                                      kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0,
                                                                      DMA ? m * k * 2 : 0x7FFFFFFF, kRsrcWord3);
  const int vw = orow * REC + lj * CB, vh = orow * REC + 256 + lj * 4, vs = orow * (1024 / G) * 2;
  // register path: chunk c = tid + j kThreads is (token c / 8, chunk c % 8), tokens past m read token 0.  DMA:
  // instruction j of wave w fills the 1 KB block b = w + (kThreads / 64) j of the stage (tokens 8 b .. 8 b + 7, 128 B
  // each), lane l writing bytes 16 l .. 16 l + 15, i.e. token 8 b + l / 8 at slot l % 8, which holds the token's chunk
  // (l % 8) ^ ((token >> 1) & 7); one offset vx[0] for all j (+ j x the block step), tokens past m reading zeros
  // through the buffer's range (m k 2 bytes)
  int vx[DMA ? 1 : XPT];
  if constexpr (DMA) {
    const int tk = 8 * wave + (lane >> 3), q = (lane & 7) ^ ((tk >> 1) & 7);  // ((tk + 64 j) >> 1) & 7 is the same
    vx[0] = ((t0 + tk) * k + 8 * q) * 2;
  } else {
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int c = tid + j * kThreads, tk = c >> 3;
      vx[j] = ((t0 + tk < m ? t0 + tk : 0) * k + 8 * (c & 7)) * 2;
    }
  }
  const bool full = t0 + kToks <= m;  // every token of the tile exists (no zero selection)
  int xsel[XPT];                      // else: per chunk, whether its token exists
#pragma unroll
  for (int j = 0; j < XPT; ++j) xsel[j] = t0 + ((tid + j * kThreads) >> 3) < m;

  struct WSlab {
    ChunkRaw<BITS> w;
  };
  struct XSlab {
    u32x4 xv[XPT];
  };
  static_assert(RING % XR == 0, "the token ring must divide the weight ring");
  WSlab rg[kRing];
  XSlab rx_[DMA ? 1 : XR];
  auto issue_w = [&](int sl, WSlab& d) __attribute__((always_inline)) {
    const int t = (sb + sl) >> 4, s16 = (sb + sl) & 15;  // tile, slab within the tile
    const int tb = t * n * REC;
    if constexpr (BITS == 4) {
      d.w.w = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, tb + s16 * 32, 0);
    } else {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 lo = __builtin_amdgcn_raw_buffer_load_b64(rw, vw, tb + s16 * 16, 0);
      const uint32_t hi = BITS == 3 ? __builtin_amdgcn_raw_buffer_load_b32(rw, vh, tb + s16 * 8, 0) : 0u;
      d.w.w = u32x4{lo[0], lo[1], hi, 0u};
    }
    d.w.s = __builtin_amdgcn_raw_buffer_load_b16(rs, vs, (t * n * (1024 / G) + (G == 128 ? s16 >> 1 : s16)) * 2, 0);
  };
  auto issue_x = [&](int sl, XSlab& d) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < XPT; ++j)
      if constexpr (!DMA) d.xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, vx[j], (sb + sl) * kSlab * 2, 0);
  };
  // DMA: slab sl's tokens into token stage xs (every wave its XPT blocks)
  auto dma_x = [&](int sl, int xs) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < XPT; ++j)
      lds_dma16(rx, lds + kXBase + xs * kXStage + (wave + (kThreads / 64) * j) * 1024,
                vx[0] + j * (kThreads / 64) * 8 * k * 2, (sb + sl) * kSlab * 2);
  };
  // (the zero selection of tokens past m happens here, at the write: selecting at the load would wait for the data)
  auto put = [&](const WSlab& d, const XSlab& dx, int stage) __attribute__((always_inline)) {
    uint8_t* base = lds + stage * kStage;
    const float s = bf2f(d.w.s);
    if constexpr (BITS == 4) {
      uint32_t nw[4];
      chunk_codes<BITS>(d.w, nw);
#pragma unroll
      for (int u = 0; u < 4; ++u) *reinterpret_cast<u32x4*>(base + swz(lr, 4 * lj + u)) = dequant8<OFF>(nw[u], s);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const HalfCodes hc = half_codes<BITS>(d.w, h);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
          *reinterpret_cast<u32x4*>(base + swz(lr, 4 * lj + 2 * h + sub)) = dequant_half<OFF>(hc, s, sub);
      }
    }
    if constexpr (DMA) return;
    uint8_t* xb = lds + kXBase + stage * kXStage;
    if (full) {
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        const int c = tid + j * kThreads;
        *reinterpret_cast<u32x4*>(xb + swz(c >> 3, c & 7)) = dx.xv[j];
      }
    } else {
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        const int c = tid + j * kThreads;
        *reinterpret_cast<u32x4*>(xb + swz(c >> 3, c & 7)) = xsel[j] ? dx.xv[j] : z;
      }
    }
  };

  // wave tiles of 64 rows x WT tokens
  constexpr int RW = kRows / 64, WT = kToks / (kThreads / 64 / RW), NJ = WT / 16;  // waves along the rows
  const int wr = (wave % RW) * 64, wtk = (wave / RW) * WT;
  const int lrow = lane & 15, lsub = lane >> 4;
  f32x4 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int stage, int xs) __attribute__((always_inline)) {
    const uint8_t* A = lds + stage * kStage;
    const uint8_t* B = lds + kXBase + xs * kXStage;
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // 32-input slices of the slab
      const int q = 4 * h + lsub;
      bf16x8 av[4], bv[NJ];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const bf16x8*>(A + swz(wr + 16 * i + lrow, q));
#pragma unroll
      for (int j = 0; j < NJ; ++j) bv[j] = *reinterpret_cast<const bf16x8*>(B + swz(wtk + 16 * j + lrow, q));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  };

  // compute(stage, xs) with put's weight half interleaved (DMA path): after each 16 MFMAs one of the next slab's four
  // words is dequantized and written, the MFMAs and that VALU work alternating in each region (a wave issues in
  // order, so VALU work placed between its MFMAs runs while they do)
  auto compute_put = [&](int stage, int xs, const WSlab& d, int wstage) __attribute__((always_inline)) {
    const uint8_t* A = lds + stage * kStage;
    const uint8_t* B = lds + kXBase + xs * kXStage;
    uint8_t* base = lds + wstage * kStage;
    uint32_t nw[4];
    if constexpr (BITS == 4) chunk_codes<BITS>(d.w, nw);
    const float sc = bf2f(d.w.s);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = 4 * h + lsub;
      HalfCodes hc;
      if constexpr (BITS != 4) hc = half_codes<BITS>(d.w, h);
      bf16x8 av[4], bv[NJ];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const bf16x8*>(A + swz(wr + 16 * i + lrow, q));
#pragma unroll
      for (int j = 0; j < NJ; ++j) bv[j] = *reinterpret_cast<const bf16x8*>(B + swz(wtk + 16 * j + lrow, q));
      // W4: the slice's MFMA run at raised wave priority, so that the SIMD's other wave, in its dequantization or
      // operand reads, yields issue slots to it (measured: W4 8-10 % faster; W3, whose unpacking is heavier, slower)
      if constexpr (BITS == 4) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ih = 0; ih < 2; ++ih) {
#pragma unroll
        for (int i = 2 * ih; i < 2 * ih + 2; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
        const int u = 2 * h + ih;
        if constexpr (BITS == 4)
          *reinterpret_cast<u32x4*>(base + swz(lr, 4 * lj + u)) = dequant8<OFF>(nw[u], sc);
        else
          *reinterpret_cast<u32x4*>(base + swz(lr, 4 * lj + u)) = dequant_half<OFF>(hc, sc, ih);
        static_for<0, 2 * NJ>([&](auto) __attribute__((always_inline)) {
          __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x0002, 3, 0);  // 1 MFMA, 3 VALU
        });
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (BITS == 4) __builtin_amdgcn_s_setprio(0);
    }
  };

  // Pipeline over slabs: two LDS stages, kRing weight register sets and XR token register sets.  Iteration sl:
  // barrier (slab sl in LDS; every wave done with slab sl - 1), issue the token loads of slab sl + XR - 1 and then the
  // weight loads of slab sl + kRing - 1 (in this order: the loads' counter is in order, and the tokens, read from L2,
  // are needed first), compute slab sl from its stage, write slab sl + 1 (dequantized) into the other stage.
  constexpr int D = kRing - 1, DX = XR - 1;
  if constexpr (DMA) {
    // Iteration sl: wait for all of this wave's loads (its token DMA of slab sl among them; the weight loads still
    // outstanding were issued a slab earlier, so this costs little, and it holds whatever order the loads were issued
    // in), barrier (every wave's DMA of slab sl landed; every wave done with slab sl - 1), DMA of slab sl + DX into
    // the token stage slab sl - 1 used, weight loads of slab sl + D, compute slab sl, write slab sl + 1's weights
    // (dequantized) into the other weight stage.
    static_assert(DX >= 1, "token DMA pipeline");
    constexpr int kVmcnt0 = 0x0F70;  // s_waitcnt immediate: vector memory counter 0, the others unconstrained
#pragma unroll
    for (int i = 0; i < DX; ++i) dma_x(i < nslab ? i : nslab - 1, i);
#pragma unroll
    for (int i = 0; i < D; ++i) issue_w(i < nslab ? i : nslab - 1, rg[i]);
    put(rg[0], rx_[0], 0);
    auto iter = [&](int sl, auto S, bool last_ok) __attribute__((always_inline)) {
      constexpr int r1 = (decltype(S)::value + 1) % kRing, rd = (decltype(S)::value + D) % kRing;
      constexpr int xc = decltype(S)::value % XR, xd = (decltype(S)::value + DX) % XR;
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      __syncthreads();
      dma_x(sl + DX < nslab ? sl + DX : nslab - 1, xd);
      issue_w(sl + D < nslab ? sl + D : nslab - 1, rg[rd]);
      if (last_ok) {
        compute_put(sl & 1, xc, rg[r1], (sl + 1) & 1);
      } else {
        compute(sl & 1, xc);
        if (sl + 1 < nslab) put(rg[r1], rx_[0], (sl + 1) & 1);
      }
    };
    int sl = 0;
    for (; sl + kRing < nslab; sl += kRing)  // every iteration here has a next slab
      static_for<0, kRing>([&](auto I) __attribute__((always_inline)) { iter(sl + decltype(I)::value, I, true); });
    static_for<0, kRing>([&](auto I) __attribute__((always_inline)) {
      if (sl + decltype(I)::value < nslab) iter(sl + decltype(I)::value, I, false);
    });
  } else {
#pragma unroll
    for (int i = 0; i < DX; ++i) issue_x(i < nslab ? i : nslab - 1, rx_[i]);
#pragma unroll
    for (int i = 0; i < D; ++i) issue_w(i < nslab ? i : nslab - 1, rg[i]);
    put(rg[0], rx_[0], 0);
    auto iter = [&](int sl, auto S) __attribute__((always_inline)) {
      constexpr int r1 = (decltype(S)::value + 1) % kRing, rd = (decltype(S)::value + D) % kRing;
      constexpr int x1 = (decltype(S)::value + 1) % XR, xd = (decltype(S)::value + DX) % XR;
      __syncthreads();
      if constexpr (DX > 0) issue_x(sl + DX < nslab ? sl + DX : nslab - 1, rx_[xd]);
      issue_w(sl + D < nslab ? sl + D : nslab - 1, rg[rd]);
      compute(sl & 1, sl & 1);
      if constexpr (DX == 0) issue_x(sl + 1 < nslab ? sl + 1 : nslab - 1, rx_[x1]);
      if (sl + 1 < nslab) put(rg[r1], rx_[x1], (sl + 1) & 1);
    };
    int sl = 0;
    for (; sl + kRing <= nslab; sl += kRing)
      static_for<0, kRing>([&](auto I) __attribute__((always_inline)) { iter(sl + decltype(I)::value, I); });
    static_for<0, kRing - 1>([&](auto I) __attribute__((always_inline)) {
      if (sl + decltype(I)::value < nslab) iter(sl + decltype(I)::value, I);
    });
  }

  // D: lane holds rows 4 (lane / 16) + e of its 16-row tile for token lane % 16
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int t = t0 + wtk + 16 * j + lrow;
    if (t >= m) continue;
    if (SPLIT) {  // the fp32 tile
      float* pr = part + ((size_t)blockIdx.y * m + t) * n;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r0 = o0 + wr + 16 * i + 4 * lsub;
        if ((n & 3) == 0 && r0 < n) {
          *reinterpret_cast<f32x4*>(pr + r0) = acc[i][j];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (r0 + e < n) pr[r0 + e] = acc[i][j][e];
        }
      }
      continue;
    }
    uint16_t* yr = y + (size_t)t * ldy;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r0 = o0 + wr + 16 * i + 4 * lsub;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (r0 + e < n) yr[r0 + e] = __builtin_bit_cast(uint16_t, (__bf16)acc[i][j][e]);
    }
  }
}

// y[t][o] = bf16(part[0][t][o] + part[1][t][o] + ... + part[S - 1][t][o]), the splits in order; 4 rows per thread
__global__ void __launch_bounds__(256) sum_splits_kernel(const float* __restrict__ part, int nsplit, int m, int n,
                                                         uint16_t* __restrict__ y, int ldy) {
  const int n4 = (n + 3) >> 2;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)m * n4) return;
  const int t = (int)(i / n4), o = (int)(i - (long long)t * n4) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if ((n & 3) == 0) {  // 16-byte partial loads, one 8-byte store
    for (int sp = 0; sp < nsplit; ++sp) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(part + ((size_t)sp * m + t) * n + o);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += v[e];
    }
    const bf16x2 lo = {(__bf16)acc[0], (__bf16)acc[1]}, hi = {(__bf16)acc[2], (__bf16)acc[3]};
    uint16_t* yo = y + (size_t)t * ldy + o;
    if ((ldy & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {  // 8-byte aligned (y may be a column offset)
      *reinterpret_cast<uint2*>(yo) = make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) yo[e] = __builtin_bit_cast(uint16_t, (__bf16)acc[e]);
    }
    return;
  }
  for (int sp = 0; sp < nsplit; ++sp) {
    const float* pr = part + ((size_t)sp * m + t) * n + o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (o + e < n) acc[e] += pr[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (o + e < n) y[(size_t)t * ldy + o + e] = __builtin_bit_cast(uint16_t, (__bf16)acc[e]);
}

template <int BITS, int G, int R, int T, int RING, int XR, bool XM, bool DMA, bool SPLIT = false>
int launch_tiles(const void* x, int m, const void* wt, const void* st, void* y, int n, int ldy, int k, hipStream_t s,
                 int nsplit = 1, float* part = nullptr) {
  const int nrt = (n + R - 1) / R, ntt = (m + T - 1) / T;
  const long long grid = XM ? ((long long)nrt * ntt + 7) / 8 * 8 : (long long)((nrt + 7) / 8) * 8 * ntt;
  if (grid > 0x7FFFFFFF) return AK_INVALID;
  hipLaunchKernelGGL((wq_gemm_kernel<BITS, G, R, T, RING, XR, XM, DMA, SPLIT>), dim3((unsigned)grid, (unsigned)nsplit), dim3(2 * R),
                     DMA ? (2 * R + XR * T) * kRowBytes : kStages * (R + T) * kRowBytes, s, static_cast<const uint16_t*>(x), m,
                     static_cast<const uint8_t*>(wt), static_cast<const uint16_t*>(st), static_cast<uint16_t*>(y), n,
                     ldy, k, nrt, ntt, part);
  if (nsplit > 1) {
    const long long items = (long long)m * ((n + 3) / 4);
    hipLaunchKernelGGL(sum_splits_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, part, nsplit, m, n,
                       static_cast<uint16_t*>(y), ldy);
  }
  return (int)hipGetLastError();
}

template <int BITS, int G>
int launch_gemm(const void* x, int m, const void* wt, const void* st, void* y, int n, int ldy, int k, hipStream_t s) {
  // 32-bit buffer offsets: the weights, scales and inputs must each stay below 2 GB
  if ((long long)kpad(k) / 1024 * n * 128 * BITS >= (1ll << 31) || (long long)m * k * 2 >= (1ll << 31))
    return AK_INVALID;
  // 256 x 256 tiles above 128 tokens where there are enough of them to fill the GPU (measured: from about 160 tiles
  // on, e.g. gate_up 55296 rows from 129 tokens, the 5120-row linears from 2048), else 128 x 128 tiles at two
  // workgroups per CU
  const long long big_tiles = (long long)((n + 255) / 256) * ((m + 255) / 256);
  // (the weights 3 slabs ahead for W4 / W2, 1 for W3: a deeper ring spills W3's registers, measured 10 % slower; W4 /
  // W2 are 5-11 % slower with 1)
  if (m > 128 && big_tiles >= 160)
    return launch_tiles<BITS, G, 256, 256, BITS == 3 ? 2 : 4, 2, true, true>(x, m, wt, st, y, n, ldy, k, s);
  // 128 x 128 tiles; where there are fewer than 384 (measured: below that, splitting k wins over the partials'
  // extra traffic), k is split across workgroups up to 512 of them (at least 8 slabs per split): fp32 partial tiles in
  // the stream's scratch after its first 4 KB (the GEMV kernels' row-range counters, which stay zero between
  // launches), summed in order by a second kernel; one pass where the scratch is not available (e.g. first use under
  // stream capture)
  const long long tiles = (long long)((n + 127) / 128) * ((m + 127) / 128);
  int nsplit = 1;
  if (tiles < 384) nsplit = (int)std::min<long long>((512 + tiles - 1) / tiles, std::min(64, k / kSlab / 8));
  float* part = nullptr;
  if (nsplit > 1) {
    if (void* z = stream_scratch(s, 4096 + (size_t)nsplit * m * n * 4))
      part = reinterpret_cast<float*>(static_cast<uint8_t*>(z) + 4096);
  }
  if (part) return launch_tiles<BITS, G, 128, 128, 4, 4, false, false, true>(x, m, wt, st, y, n, ldy, k, s, nsplit, part);
  return launch_tiles<BITS, G, 128, 128, 4, 4, false, false>(x, m, wt, st, y, n, ldy, k, s);
}

}  // namespace
}  // namespace agq

// No single counterpart in the reference: the fusion of ak_wq_dequant_kt_rows (kernels/src/w4_gemv.cu:877-895) and
// ak_bf16_linear_f32reduce_ld (kernels/src/bf16_linear.cu:68-80), the pair the model's linear() runs above 128 tokens
// (kernels/m1/m1_model.cu:1876-1897).
extern "C" int ak_wq_gemm_kt(int bits, const void* x, int m, const void* wt, const void* st, void* y, int n, int ldy,
                             int k, int group, void* stream) {
  if (!x || !wt || !st || !y || m < 1 || n < 1 || k < 1 || (group != 64 && group != 128) || k % group != 0)
    return AK_INVALID;
  const int ld = ldy ? ldy : n;
  if (ld < n) return AK_INVALID;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (bits * 1000 + group) {
    case 4128: return agq::launch_gemm<4, 128>(x, m, wt, st, y, n, ld, k, s);
    case 4064: return agq::launch_gemm<4, 64>(x, m, wt, st, y, n, ld, k, s);
    case 3128: return agq::launch_gemm<3, 128>(x, m, wt, st, y, n, ld, k, s);
    case 3064: return agq::launch_gemm<3, 64>(x, m, wt, st, y, n, ld, k, s);
    case 2128: return agq::launch_gemm<2, 128>(x, m, wt, st, y, n, ld, k, s);
    case 2064: return agq::launch_gemm<2, 64>(x, m, wt, st, y, n, ld, k, s);
    default: return AK_INVALID;
  }
}
