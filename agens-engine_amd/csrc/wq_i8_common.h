// Device helpers shared by the integer-MFMA GEMV kernels (wq_i8.hip: any m; wq_i8m1.hip: m = 1).
// The numerics they implement are described at the top of wq_i8.hip.
#pragma once
#include "wq_common.h"
#include "wq_silu.h"

namespace agq {

struct I8Args {
  Segs segs;
  const uint16_t* x;
  int m, k;
  int nquad, P;   // quads of the padded k, stripes
  int qpt;        // quads per 1024-input tile (2 for group 128, 4 for group 64)
  int nb;         // quads per LDS batch (any-m kernel)
  int wg_end[4];  // m = 1 kernel: workgroups of segments 0..i (each workgroup serves one segment)
  float* part;    // split-K launches: stripe partials [P][tokens][rows] and, at cnt, one counter per row range
  int* cnt;
  int act = 0;    // 1: x is the merged gate_up [m][2k] and the activations are SiLU(gate) * up (wq_silu.h)
  // group-128 kernels (set_tile_stripes): the multiplier of x / P (0 for P = 1) and bit t set when 1024-input tile t
  // ends a stripe (up to 64 tiles)
  unsigned pmul = 0;
  unsigned long long ends = 0;
  // chained launches: a tagged copy of each segment's outputs for the next step (32-bit words bf16 | tag << 16, laid
  // out as y), and the tagged copy this step's activations are read from (written by the step before it)
  uint32_t* ytg[4] = {nullptr, nullptr, nullptr, nullptr};
  const uint32_t* xtg = nullptr;
};

// The P (<= 8) stripe partials of one output of a split-K launch, at float offsets off + q * stride (q < P) of base,
// written by other workgroups with device-coherent stores: loaded device-coherently (sc1: not served from a stale L2
// line) all at once, then added in stripe order from stripe 0.  One dependent round trip instead of P.
__device__ __forceinline__ float sum_stripe_partials(const float* base, size_t off, size_t stride, int P) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7FFFFFFF, 0x00020000);
  float v[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    v[q] = q < P ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)((off + q * stride) * 4), 0, 16)) : 0.f;
  float y = v[0];
#pragma unroll
  for (int q = 1; q < 8; ++q)
    if (q < P) y += v[q];
  return y;
}

// The same for U outputs at once: the loads of all of them are requested before any sum.
template <int U>
__device__ __forceinline__ void sum_stripe_partials_n(const float* base, const size_t (&off)[U], size_t stride, int P,
                                                      float (&y)[U]) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7FFFFFFF, 0x00020000);
  float v[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int q = 0; q < 8; ++q)
      v[u][q] = q < P ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)((off[u] + q * stride) * 4), 0, 16))
                      : 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    y[u] = v[u][0];
#pragma unroll
    for (int q = 1; q < 8; ++q)
      if (q < P) y[u] += v[u][q];
  }
}

// Stripes are contiguous runs of whole 1024-input tiles: with nt = nquad / qpt tiles, P = min(8, nt) stripes and stripe
// p = tiles [p * nt / P, (p + 1) * nt / P), i.e. quads [qpt * (p * nt / P), qpt * ((p + 1) * nt / P)).
__host__ __device__ inline int stripe_count(int nquad, int qpt) { return nquad / qpt < 8 ? nquad / qpt : 8; }
// x / d for 0 <= x < 2^23 and 1 <= d <= 8 by a multiply with ceil(2^32 / d) (exact in that range: the error term
// x (M d - 2^32) / (d 2^32) < 2^-9 stays below the distance 1 / d of x / d to the next integer); a runtime 32-bit
// division is a long instruction sequence on the GPU, and the scalar unit running it is shared by the CU's waves
__host__ __device__ inline unsigned upto8_mul(int d) {
  return d == 2 ? 2147483649u : d == 3 ? 1431655766u : d == 4 ? 1073741825u : d == 5 ? 858993460u
       : d == 6 ? 715827883u : d == 7 ? 613566757u : 536870913u;
}
__host__ __device__ inline int div_upto8(int x, int d) {
  return d == 1 ? x : (int)(((unsigned long long)(unsigned)x * upto8_mul(d)) >> 32);
}
// first quad of stripe p (p <= P <= 8, fewer than 2^20 tiles)
__host__ __device__ inline int stripe_begin(int p, int nquad, int P, int qpt) {
  return qpt * div_upto8(p * (nquad / qpt), P);
}
// x / P with the launch's multiplier (branch-free on the device: a selection on P costs scalar branches)
__device__ __forceinline__ int div_by_p(int x, const I8Args& a) {
  return (int)(((unsigned long long)(unsigned)x * a.pmul) >> 32) + (a.P == 1 ? x : 0);
}
// P, its multiplier and the stripe-end mask of a group-128 launch (qpt 2) from nquad
inline void set_tile_stripes(I8Args& a) {
  a.P = stripe_count(a.nquad, 2);
  a.pmul = a.P == 1 ? 0u : upto8_mul(a.P);
  const int nt = a.nquad / 2;
  a.ends = 0;
  for (int p = 0; p < a.P && nt <= 64; ++p) a.ends |= 1ull << (stripe_begin(p + 1, a.nquad, a.P, 2) / 2 - 1);
}

namespace {

__device__ __forceinline__ uint32_t byte_of(uint32_t v, int j) { return (v >> (8 * j)) & 0xFFu; }

template <int BITS>
constexpr int code_offset() { return BITS == 4 ? 8 : BITS == 3 ? 4 : 2; }

// -OFF in every byte: the constant B operand that turns sum(d * n) into sum(d * q)
template <int BITS>
constexpr int neg_off_bytes() { return BITS == 4 ? (int)0xF8F8F8F8u : BITS == 3 ? (int)0xFCFCFCFCu : (int)0xFEFEFEFEu; }

template <int BITS>
struct Raw;
template <>
struct Raw<4> { uint4 w; };
template <>
struct Raw<3> { uint2 lo; uint32_t hi; };
template <>
struct Raw<2> { uint2 lo; };

template <int BITS>
__device__ __forceinline__ Raw<BITS> load_raw(const void* __restrict__ wt, size_t rec, int c) {
  Raw<BITS> r;
  if constexpr (BITS == 4) {
    r.w = ld_stream(reinterpret_cast<const uint4*>(wt) + rec * 32 + c);
  } else {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(wt) + rec * (32 * BITS);
    r.lo = ld_stream2(reinterpret_cast<const uint2*>(p) + c);
    if constexpr (BITS == 3) r.hi = ld_stream1(p + 64 + c);
  }
  return r;
}

// The two B operands (16 int8 codes each) of one lane chunk.  Input o (0..31) of the chunk lands at
//   W4: half o % 2, VGPR o / 8, byte (o % 8) / 2;  W2: half o / 16, VGPR o % 4, byte (o % 16) / 4;
//   W3: half (o % 8) / 4, VGPR o % 4, byte o / 8.
template <int BITS>
__device__ __forceinline__ void make_b(const Raw<BITS>& r, i32x4& b0, i32x4& b1) {
  if constexpr (BITS == 4) {
    const uint32_t w[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      b0[v] = (int)(w[v] & 0x0F0F0F0Fu);
      b1[v] = (int)((w[v] >> 4) & 0x0F0F0F0Fu);
    }
  } else if constexpr (BITS == 2) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      b0[s] = (int)((r.lo.x >> (2 * s)) & 0x03030303u);
      b1[s] = (int)((r.lo.y >> (2 * s)) & 0x03030303u);
    }
  } else {
    const uint32_t L0 = r.lo.x, L1 = r.lo.y, H = r.hi;
    // bytes m of P0 / P1 hold the 2-bit fields of inputs 8m .. 8m+3 / 8m+4 .. 8m+7 (bytes 0, 2 / 1, 3 of L0 and L1)
    const uint32_t P0 = __builtin_amdgcn_perm(L1, L0, 0x06040200u), P1 = __builtin_amdgcn_perm(L1, L0, 0x07050301u);
    // code byte = 2-bit field | third bit << 2; the third bits of inputs 8m + t sit in bit t of byte m of H, moved to
    // bit 2 with one shift and one mask, then merged by one and-or (31 operations per lane chunk)
    b0[0] = (int)((P0 & 0x03030303u) | ((H << 2) & 0x04040404u));
    b0[1] = (int)(((P0 >> 2) & 0x03030303u) | ((H << 1) & 0x04040404u));
    b0[2] = (int)(((P0 >> 4) & 0x03030303u) | (H & 0x04040404u));
    b0[3] = (int)(((P0 >> 6) & 0x03030303u) | ((H >> 1) & 0x04040404u));
    b1[0] = (int)((P1 & 0x03030303u) | ((H >> 2) & 0x04040404u));
    b1[1] = (int)(((P1 >> 2) & 0x03030303u) | ((H >> 3) & 0x04040404u));
    b1[2] = (int)(((P1 >> 4) & 0x03030303u) | ((H >> 4) & 0x04040404u));
    b1[3] = (int)(((P1 >> 6) & 0x03030303u) | ((H >> 5) & 0x04040404u));
  }
}

// The group's limb sums -> fp32: T = D2 * 256 + D1 (exact int32), gsum = fmaf((float)T, 256, (float)D0), i.e.
// fp32_rn(GS) whenever |T| < 2^24 (always but for adversarial data).  The caller multiplies by scale * 2^(E - 148).
__device__ __forceinline__ float group_sum_f32(const i32x4& d) {
  const int t = d[2] * 256 + d[1];
  return fmaf((float)t, 256.0f, (float)d[0]);
}

// The activation scale of a group as fp32 bits, from the group's largest bf16 magnitude pattern mx (sign cleared):
// 2^(E - 148) with E = mx >> 7 the largest exponent field; a group holding a NaN (mx above the Inf pattern 0x7F80):
// NaN; a group holding an Inf but no NaN: +Inf.  In a non-finite group every finite input converts to 0 and every Inf
// to its sign (+-1, see x_int), so the group sum S is the sum of sign(x) * q over the Inf inputs and the
// group adds S * scale * Inf: +-Inf, or NaN where S = 0 -- the fp32 path's value wherever the group's Inf products
// share one sign (the fp32 path gives NaN for products of both signs, where S may be nonzero).
__device__ __forceinline__ int act_scale_bits(int mx) {
  return mx > 0x7F80 ? 0x7FC00000 : mx == 0x7F80 ? 0x7F800000 : __float_as_int(ldexpf(1.0f, (mx >> 7) - 148));
}

// x_int of one bf16 input of a group with largest exponent field e: trunc(x * 2^(148 - e)), exact (|x_int| < 2^22).
// A non-finite group (e = 255): +-1 for +-Inf and 0 for every finite input (scaled by 2^-200 instead, every finite bf16
// truncates to 0, an Inf stays infinite and is clamped to its sign); a NaN group's values do not matter, its activation
// scale is NaN.  XiScale holds the group's exponent shift and clamp bound.
struct XiScale {
  int sh;
  float lim;
};
__device__ __forceinline__ XiScale xi_scale(int e) {
  return e == 255 ? XiScale{-200, 1.0f} : XiScale{148 - e, 16777216.0f};
}
__device__ __forceinline__ int x_int(uint32_t b16, XiScale s) {
  return (int)__builtin_amdgcn_fmed3f(ldexpf(bf2f(b16), s.sh), -s.lim, s.lim);
}

// Reductions over aligned groups of L lanes (L = 2, 4, 8 or 16) with DPP: two quad swaps, then the half-row and the
// row mirrors (each step pairs every lane with one holding the other half of its group's partial results).
template <int L, bool MAX>
__device__ __forceinline__ int dpp_group_reduce(int v) {
  auto step = [&](int o) { return MAX ? max(v, o) : v + o; };
  v = step(__builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));                    // quad_perm [1,0,3,2]
  if constexpr (L >= 4) v = step(__builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  if constexpr (L >= 8) v = step(__builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false)); // row_half_mirror
  if constexpr (L >= 16) v = step(__builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false)); // row_mirror
  return v;
}

// One group's activation limbs from 8 consecutive bf16 inputs per lane, LPU lanes per group: the group's largest
// magnitude pattern mx (all LPU lanes; the exponent field E = mx >> 7) and, per input, x_int = trunc(x * 2^(148 - E))
// with its three limb-byte sources.
template <int LPU>
__device__ __forceinline__ int group_limbs(const uint4 v, uint32_t (&t0)[8], uint32_t (&t1)[8], uint32_t (&t2)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  int mx = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) mx = max(mx, max((int)(w[i] & 0x7FFFu), (int)((w[i] >> 16) & 0x7FFFu)));
  mx = dpp_group_reduce<LPU, true>(mx);
  const XiScale xs = xi_scale(mx >> 7);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int xi = x_int((w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu, xs);
    t0[i] = (uint32_t)xi;          // limb 0 = byte 0
    t1[i] = (uint32_t)xi + 0x80u;    // limb 1 = byte 1
    t2[i] = (uint32_t)xi + 0x8080u;  // limb 2 = byte 2
  }
  return mx;
}

// Writes the limb bytes of inputs o0 .. o0+7 of a lane chunk: dst points at (chunk, half 0, limb 0) of the LDS operand
// layout, half_stride = bytes between half 0 and half 1 (limb rows are 16 bytes apart).
template <int BITS>
__device__ __forceinline__ void store_limbs(uint8_t* dst, size_t half_stride, int o0, const uint32_t (&t0)[8],
                                            const uint32_t (&t1)[8], const uint32_t (&t2)[8]) {
  if constexpr (BITS == 4) {
    // word v = o0 / 8: even inputs -> half 0 bytes 0..3, odd -> half 1
    const int v4 = o0 >> 3;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int limb = 0; limb < 3; ++limb) {
        const uint32_t* t = limb == 0 ? t0 : limb == 1 ? t1 : t2;
        const uint32_t d = byte_of(t[hf], limb) | (byte_of(t[hf + 2], limb) << 8) | (byte_of(t[hf + 4], limb) << 16) |
                           (byte_of(t[hf + 6], limb) << 24);
        *reinterpret_cast<uint32_t*>(dst + hf * half_stride + limb * 16 + 4 * v4) = d;
      }
  } else if constexpr (BITS == 2) {
    // half o0 / 16, VGPR i % 4, byte 2 * ((o0 / 8) % 2) + i / 4
    const int hf = o0 >> 4, bb = 2 * ((o0 >> 3) & 1);
#pragma unroll
    for (int limb = 0; limb < 3; ++limb) {
      const uint32_t* t = limb == 0 ? t0 : limb == 1 ? t1 : t2;
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) {
        const uint16_t d = (uint16_t)(byte_of(t[vv], limb) | (byte_of(t[vv + 4], limb) << 8));
        *reinterpret_cast<uint16_t*>(dst + hf * half_stride + limb * 16 + 4 * vv + bb) = d;
      }
    }
  } else {
    // W3: half i / 4, VGPR i % 4, byte o0 / 8
    const int bb = o0 >> 3;
#pragma unroll
    for (int limb = 0; limb < 3; ++limb) {
      const uint32_t* t = limb == 0 ? t0 : limb == 1 ? t1 : t2;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        dst[(i >> 2) * half_stride + limb * 16 + 4 * (i & 3) + bb] = (uint8_t)byte_of(t[i], limb);
    }
  }
}



// The inputs a lane converts.  A unit is a group of 128 inputs of one token held by 16 lanes (sub = lane of the group,
// chunk sub / 4 of the group, lq = sub % 4 within the chunk); each lane holds four pairs of adjacent inputs, pair c
// (c < 4) at element offset unit_pair_offset(sub, c) of the group.  The pairs are chosen so that a lane's limb bytes
// fill whole dwords of the MFMA A operand, whose input order follows make_b:
//   W4: 8 consecutive inputs 8 lq .. 8 lq + 7 (even inputs -> half 0, odd -> half 1, dword lq of each);
//   W3: inputs 8 c + 2 lq (+1): half lq / 2, dwords 2 (lq % 2) (low input of each pair) and +1 (high), byte c;
//   W2: inputs 16 (lq / 2) + 2 (lq % 2) + 4 c (+1): the same half, dwords and bytes.
template <int BITS>
__device__ __forceinline__ int unit_pair_offset(int sub, int c) {
  const int l = sub & 3, base = 32 * (sub >> 2);
  return BITS == 4 ? base + 8 * l + 2 * c : BITS == 3 ? base + 2 * l + 8 * c : base + 16 * (l >> 1) + 2 * (l & 1) + 4 * c;
}
// the lane's four pairs of the group starting at g (generic pointer)
template <int BITS>
__device__ __forceinline__ uint4 load_unit(const uint16_t* g, int sub) {
  if constexpr (BITS == 4) {
    return *reinterpret_cast<const uint4*>(g + unit_pair_offset<4>(sub, 0));
  } else {
    uint32_t w[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) w[c] = *reinterpret_cast<const uint32_t*>(g + unit_pair_offset<BITS>(sub, c));
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// One unit of a group-128 activation image (the lane's pairs in v, as load_unit gives them): computes what
// group_limbs, store_limbs and the limb sums do, with fewer operations:
//   - the group's largest exponent field is the exponent of the largest magnitude (packed 16-bit maxima of the sign-
//     cleared patterns; NaN / Inf patterns order above every finite one, as their exponent fields do);
//   - the limb dwords are gathered with byte permutes, their sums taken from the same dwords (sdot4), and written
//     whole (W4: one dword per half and limb; W2 / W3: one 8-byte store per limb);
//   - the limb-0 and limb-1 sums of the group share one packed reduction (|sum| <= 128 * 128 < 2^15).
// dst points at (chunk, half 0, limb 0) of the LDS operand layout (limb rows 16 bytes apart), half_stride = bytes
// between half 0 and half 1.  Returns the group's largest magnitude pattern (act_scale_bits' argument); d0..d2 = the
// group's limb sums (every lane of the unit).  store = false: nothing is written.
template <int BITS>
__device__ __forceinline__ int convert_unit(const uint4 v, uint8_t* dst, size_t half_stride, int lq, bool store,
                                            int& d0, int& d1, int& d2) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  auto mag = [](uint32_t w) {
    const uint32_t m = w & 0x7FFF7FFFu;
    return __builtin_bit_cast(u16x2, m);
  };
  const u16x2 mx = __builtin_elementwise_max(__builtin_elementwise_max(mag(v.x), mag(v.y)),
                                             __builtin_elementwise_max(mag(v.z), mag(v.w)));
  const int mxg = dpp_group_reduce<16, true>(max((int)mx.x, (int)mx.y));
  const XiScale xs = xi_scale(mxg >> 7);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t t0[8], t1[8], t2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int xi = x_int((w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu, xs);
    t0[i] = (uint32_t)xi;
    t1[i] = (uint32_t)xi + 0x80u;
    t2[i] = (uint32_t)xi + 0x8080u;
  }
  int sums[3];
#pragma unroll
  for (int limb = 0; limb < 3; ++limb) {
    const uint32_t* t = limb == 0 ? t0 : limb == 1 ? t1 : t2;
    const uint32_t sel = (uint32_t)limb | ((uint32_t)(4 + limb) << 8) | 0x0C0C0000u;  // [a.byte l, b.byte l, 0, 0]
    // W4: half hf = inputs hf, hf + 2, hf + 4, hf + 6; W2 / W3: dword 0 = the pairs' low inputs 0, 2, 4, 6, dword 1 =
    // their high inputs: the same two gathers
    uint32_t d[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint32_t lo = __builtin_amdgcn_perm(t[hf + 2], t[hf], sel);
      const uint32_t hi = __builtin_amdgcn_perm(t[hf + 6], t[hf + 4], sel);
      d[hf] = lo | (hi << 16);
    }
    sums[limb] = __builtin_amdgcn_sdot4((int)d[1], 0x01010101, __builtin_amdgcn_sdot4((int)d[0], 0x01010101, 0, false),
                                        false);
    if (store) {
      if constexpr (BITS == 4) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) *reinterpret_cast<uint32_t*>(dst + hf * half_stride + limb * 16 + 4 * lq) = d[hf];
      } else {
        *reinterpret_cast<uint2*>(dst + (lq >> 1) * half_stride + limb * 16 + 8 * (lq & 1)) = make_uint2(d[0], d[1]);
      }
    }
  }
  const int p01 = dpp_group_reduce<16, false>(sums[0] + (int)((uint32_t)sums[1] << 16));
  d2 = dpp_group_reduce<16, false>(sums[2]);
  d0 = (int)(short)(p01 & 0xFFFF);
  d1 = (p01 - d0) >> 16;
  return mxg;
}

}  // namespace
}  // namespace agq
