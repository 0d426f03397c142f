// Device helpers of the kernels whose items are 16 rows x one quad (512 inputs) of the KT records (wq_i8mt.hip,
// wq_mm.hip): the raw words of an item, the lane exchange that turns them into per-group lane chunks, and the
// segment-field selects.
#pragma once
#include "wq_i8_common.h"

namespace agq {
namespace {

// one item of one lane: the raw weight words of the quad's four groups (W2 / W3: before the lane exchange) and the
// scales of its row for the four groups
template <int BITS>
struct QuadRaw;
template <>
struct QuadRaw<4> { uint4 w[4]; uint2 s; };
template <>
struct QuadRaw<3> { uint4 lo[2]; uint2 hi[2]; uint2 s; };
template <>
struct QuadRaw<2> { uint4 lo[2]; uint2 s; };

// Item loads cover whole 128-byte lines: the lanes of a column pair (c even, c + 1) load the same row, the even lane
// the first 64 bytes of the line and the odd lane the second, so one instruction reads 8 rows' lines whole (instead of
// half of each of 16 rows' lines: half-line loads stream about a quarter slower).  Load e of a pair is row
// 2 (c >> 1) + e of the block; quad_pair_rows then gives each lane its own row back: lane c keeps the half of its own
// row and receives the other half from lane c ^ 1 (one DPP swap per dword pair).
//   W4: load 2 L + e = line L of the quad's two lines, bytes (c & 1) 64 + 16 h -> chunk h of group 2 L + (c & 1);
//   W2 / W3 two-bit planes: load e = the quad's line, bytes (c & 1) 64 + 8 cp -> the chunk pair of groups
//     2 (c & 1) + {0, 1} (the permlane16_swap of quad_groups follows);
//   W3 third-bit plane: load e = the quad's 64 bytes, bytes (c & 1) 32 + 4 cp, the same way.
// Per-lane parts of the offsets (rec: bytes per row and tile; cp = 4 (h & 1) + 2 (h >> 1)):
__device__ __forceinline__ int quad_vo_w(int bits, int c, int h, int rec) {
  const int cp = 4 * (h & 1) + 2 * (h >> 1);
  return 2 * (c >> 1) * rec + (c & 1) * 64 + (bits == 4 ? h * 16 : cp * 8);
}
__device__ __forceinline__ int quad_vo_h(int c, int h, int rec) {
  const int cp = 4 * (h & 1) + 2 * (h >> 1);
  return 2 * (c >> 1) * rec + 256 + (c & 1) * 32 + cp * 4;
}

// a = load 0, b = load 1 of a dword -> a = the even-position value of the lane's own row, b = the odd-position one
__device__ __forceinline__ void pair_rows(uint32_t& a, uint32_t& b, bool odd) {
  const uint32_t v = odd ? a : b;  // what the partner lane needs
  const uint32_t r = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true);  // quad_perm [1, 0, 3, 2]
  a = odd ? r : a;
  b = odd ? b : r;
}
__device__ __forceinline__ void pair_rows4(uint4& a, uint4& b, bool odd) {
  pair_rows(a.x, b.x, odd);
  pair_rows(a.y, b.y, odd);
  pair_rows(a.z, b.z, odd);
  pair_rows(a.w, b.w, odd);
}

// the raw words of a lane's own row from the pair loads (odd: c & 1); the scales are loaded per row already
template <int BITS>
__device__ __forceinline__ void quad_pair_rows(QuadRaw<BITS>& q, bool odd) {
  if constexpr (BITS == 4) {
    pair_rows4(q.w[0], q.w[1], odd);
    pair_rows4(q.w[2], q.w[3], odd);
  } else {
    pair_rows4(q.lo[0], q.lo[1], odd);
    if constexpr (BITS == 3) {
      pair_rows(q.hi[0].x, q.hi[1].x, odd);
      pair_rows(q.hi[0].y, q.hi[1].y, odd);
    }
  }
}

__device__ __forceinline__ uint2 swap16(uint32_t a, uint32_t b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  return make_uint2(r[0], r[1]);
}

// the raw operand of group s of the quad (after the lane exchange of its pair)
template <int BITS>
__device__ __forceinline__ void quad_groups(const QuadRaw<BITS>& q, Raw<BITS> (&r)[4]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int s = 0; s < 4; ++s) r[s].w = q.w[s];
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint2 a = swap16(q.lo[j].x, q.lo[j].z), b = swap16(q.lo[j].y, q.lo[j].w);
      r[2 * j].lo = make_uint2(a.x, b.x);
      r[2 * j + 1].lo = make_uint2(a.y, b.y);
      if constexpr (BITS == 3) {
        const uint2 hh = swap16(q.hi[j].x, q.hi[j].y);
        r[2 * j].hi = hh.x;
        r[2 * j + 1].hi = hh.y;
      }
    }
  }
}

template <typename T>
__device__ __forceinline__ T pick4(int i, T v0, T v1, T v2, T v3) {
  return i == 0 ? v0 : i == 1 ? v1 : i == 2 ? v2 : v3;
}
#define AK_PICK(i, arr) pick4((i), (arr)[0], (arr)[1], (arr)[2], (arr)[3])
static_assert(kMaxSegs == 4, "segment selects cover four segments");

}  // namespace
}  // namespace agq
