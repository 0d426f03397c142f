// Prefill GEMM straight from the KT weights, gfx950: y[t][o] (row stride ldy) = bf16(sum_i x[t][i] * w[o][i]) with
// w[o][i] = bf16_rn(q * scale) -- the values ak_wq_dequant_kt_rows writes, bit for bit -- and fp32 accumulation.
//
// The reference's prefill route (kernels/m1/m1_model.cu:1876-1897) dequantizes a tile of output rows into a bf16
// scratch (2 bytes per weight written, then read again) and runs a library GEMM (ak_bf16_linear_f32reduce_ld,
// kernels/src/bf16_linear.cu:68-92).  Here the KT records are read once per token tile, expanded to bf16 in registers
// and written to LDS, and v_mfma_f32_16x16x32_bf16 consumes them there: no scratch, no second pass over the weights.
//
// Tiles: a workgroup (256 threads, 4 waves; two per CU) owns 128 output rows x 128 tokens and walks k in 64-input
// slabs:
//   - loads, kRing - 1 slabs ahead in a ring of registers: thread (row tid / 2, half tid % 2) loads its lane chunk of
//     the slab from the row's KT record (W4 16 B, W3 8 + 4 B, W2 8 B) and the group's scale; the inputs are 1024
//     16-byte chunks per slab, 8 consecutive threads reading one token's 128 bytes.  Raw buffer loads with a per-lane
//     offset fixed for the kernel and a scalar per-slab offset keep address arithmetic off the vector unit; no load
//     sits under a branch (the compiler's wait counts stay exact, so the ring stays full);
//   - LDS (two stages of 16 KB weights + 16 KB inputs): rows / tokens of 64 bf16 (128 B); the 16-byte chunk q of row
//     r sits at slot q ^ ((r >> 1) & 7), so the 16 rows of one MFMA operand read hit 16 distinct 16-byte bank slots;
//   - compute: wave w owns rows 64 (w & 1) .. +63 and tokens 64 (w >> 1) .. +63, 4 x 4 MFMA tiles of 16 x 16, two
//     32-input slices per slab; lane l reads 8 inputs 8 (l / 16) .. of its slice for row / token l % 16 (the same
//     input-to-slot map for weights and tokens, which is all an MFMA needs).
// The accumulation order is this kernel's own (fp32 MFMA sums over 32 inputs, slabs in order): results agree with the
// reference's cuBLAS route and with the oracle's dequantized weights times x in fp64 within fp32-accumulation error.
// Grid: row tile major with the token tiles of a row tile 8 workgroups apart (same XCD: workgroup i runs on XCD
// i % 8), so the token tiles of one row tile share its weights through that XCD's L2.
#include <type_traits>

#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// a workgroup: kRows output rows x kToks tokens, 64-input slabs, wave tiles of 64 x 64 (kRows / 64 x 2 waves)
constexpr int kRows = 128, kToks = 128, kSlab = 64, kThreads = kRows * 2, kStages = 2, kRing = 4;
constexpr int kRowBytes = kSlab * 2;                 // one row / token of a slab in LDS
constexpr int kStage = (kRows + kToks) * kRowBytes;
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

template <int BITS, int G>
__global__ void __launch_bounds__(kThreads, 2) wq_gemm_kernel(const uint16_t* __restrict__ x, int m,
                                                              const uint8_t* __restrict__ wt,
                                                              const uint16_t* __restrict__ st,
                                                              uint16_t* __restrict__ y, int n, int ldy, int k,
                                                              int ntok_tiles) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int OFF = BITS == 4 ? 8 : BITS == 3 ? 4 : 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // workgroup -> (row tile, token tile): blocks of 8 row tiles x all token tiles, the token tiles of a row tile 8 apart
  const int b = blockIdx.x, grp = b / (8 * ntok_tiles), in = b - grp * 8 * ntok_tiles;
  const int rt = grp * 8 + (in & 7), tt = in >> 3;
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
  const int nslab = k / kSlab;
  // buffer loads: a per-lane offset fixed for the whole loop plus a per-slab scalar offset (no address arithmetic on
  // the vector unit in the loop); every buffer is below 2 GB (checked by the launcher)
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wt), (short)0, 0x7FFFFFFF,
                                                                      kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(st), (short)0, 0x7FFFFFFF,
                                                                      kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0, 0x7FFFFFFF,
                                                                      kRsrcWord3);
  const int vw = orow * REC + lj * CB, vh = orow * REC + 256 + lj * 4, vs = orow * (1024 / G) * 2;
  int vx[XPT];
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int c = tid + j * kThreads, tk = c >> 3;
    vx[j] = ((t0 + tk < m ? t0 + tk : 0) * k + 8 * (c & 7)) * 2;
  }
  const bool full = t0 + kToks <= m;  // every token of the tile exists (no zero selection)
  int xsel[XPT];                      // else: per chunk, whether its token exists
#pragma unroll
  for (int j = 0; j < XPT; ++j) xsel[j] = t0 + ((tid + j * kThreads) >> 3) < m;

  struct Slab {
    ChunkRaw<BITS> w;
    u32x4 xv[XPT];
  };
  Slab rg[kRing];
  auto issue = [&](int sl, Slab& d) __attribute__((always_inline)) {
    const int t = sl >> 4, s16 = sl & 15;  // tile, slab within the tile
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
#pragma unroll
    for (int j = 0; j < XPT; ++j) d.xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, vx[j], sl * kSlab * 2, 0);
  };
  // (the zero selection of tokens past m happens here, at the write: selecting at the load would wait for the data)
  auto put = [&](const Slab& d, int stage) __attribute__((always_inline)) {
    uint8_t* base = lds + stage * kStage;
    uint32_t nw[4];
    chunk_codes<BITS>(d.w, nw);
    const float s = bf2f(d.w.s);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      *reinterpret_cast<u32x4*>(base + swz(lr, 4 * lj + u)) = dequant8<OFF>(nw[u], s);
    }
    uint8_t* xb = base + kRows * kRowBytes;
    if (full) {
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        const int c = tid + j * kThreads;
        *reinterpret_cast<u32x4*>(xb + swz(c >> 3, c & 7)) = d.xv[j];
      }
    } else {
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        const int c = tid + j * kThreads;
        *reinterpret_cast<u32x4*>(xb + swz(c >> 3, c & 7)) = xsel[j] ? d.xv[j] : z;
      }
    }
  };

  // wave tiles of 64 rows x 64 tokens
  constexpr int RW = kRows / 64;  // waves along the rows
  const int wr = (wave % RW) * 64, wtk = (wave / RW) * 64;
  const int lrow = lane & 15, lsub = lane >> 4;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int stage) __attribute__((always_inline)) {
    const uint8_t* A = lds + stage * kStage;
    const uint8_t* B = A + kRows * kRowBytes;
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // 32-input slices of the slab
      const int q = 4 * h + lsub;
      bf16x8 av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        av[i] = *reinterpret_cast<const bf16x8*>(A + swz(wr + 16 * i + lrow, q));
        bv[i] = *reinterpret_cast<const bf16x8*>(B + swz(wtk + 16 * i + lrow, q));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  };

  // Pipeline over slabs: two LDS stages and kRing register sets.  Iteration sl: barrier (slab sl in LDS; every wave
  // done with slab sl - 1), issue the loads of slab sl + kRing - 1, compute slab sl from its stage, write slab sl + 1
  // (dequantized) into the other stage.
  constexpr int D = kRing - 1;
#pragma unroll
  for (int i = 0; i < D; ++i) issue(i < nslab ? i : nslab - 1, rg[i]);
  put(rg[0], 0);
  auto iter = [&](int sl, auto S) __attribute__((always_inline)) {
    constexpr int r1 = (decltype(S)::value + 1) % kRing, rd = (decltype(S)::value + D) % kRing;
    __syncthreads();
    issue(sl + D < nslab ? sl + D : nslab - 1, rg[rd]);
    compute(sl & 1);
    if (sl + 1 < nslab) put(rg[r1], (sl + 1) & 1);
  };
  int sl = 0;
  for (; sl + kRing <= nslab; sl += kRing)
    static_for<0, kRing>([&](auto I) __attribute__((always_inline)) { iter(sl + decltype(I)::value, I); });
  static_for<0, kRing - 1>([&](auto I) __attribute__((always_inline)) {
    if (sl + decltype(I)::value < nslab) iter(sl + decltype(I)::value, I);
  });

  // D: lane holds rows 4 (lane / 16) + e of its 16-row tile for token lane % 16
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = t0 + wtk + 16 * j + lrow;
    if (t >= m) continue;
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

template <int BITS, int G>
int launch_gemm(const void* x, int m, const void* wt, const void* st, void* y, int n, int ldy, int k, hipStream_t s) {
  const int nrt = (n + kRows - 1) / kRows, ntt = (m + kToks - 1) / kToks;
  // 32-bit buffer offsets: the weights, scales and inputs must each stay below 2 GB
  if ((long long)kpad(k) / 1024 * n * 128 * BITS >= (1ll << 31) || (long long)m * k * 2 >= (1ll << 31))
    return AK_INVALID;
  const long long grid = (long long)((nrt + 7) / 8) * 8 * ntt;
  if (grid > 0x7FFFFFFF) return AK_INVALID;
  hipLaunchKernelGGL((wq_gemm_kernel<BITS, G>), dim3((unsigned)grid), dim3(kThreads), kStages * kStage, s,
                     static_cast<const uint16_t*>(x), m, static_cast<const uint8_t*>(wt),
                     static_cast<const uint16_t*>(st), static_cast<uint16_t*>(y), n, ldy, k, ntt);
  return (int)hipGetLastError();
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
