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
