// SiLU(gate) * up of one bf16 pair: the one definition of the value shared by ak_silu_mul and the GEMV kernels that
// apply it to their activations as they load them.  Reference expression (kernels/src/fastmath/silu_mul.cu:24-27):
// bf16(g / (1 + exp(-g)) * u) in fp32, written in the same order; exp is the device library's expf, the division an
// fp32 division.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wq_common.h"

namespace agq {

__device__ __forceinline__ float silu_mul_f32(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// two packed bf16 (low half first) of gate and up -> two packed bf16 products
__device__ __forceinline__ uint32_t silu_mul_pair(uint32_t g, uint32_t u) {
  const float g0 = __uint_as_float(g << 16), g1 = __uint_as_float(g & 0xFFFF0000u);
  const float u0 = __uint_as_float(u << 16), u1 = __uint_as_float(u & 0xFFFF0000u);
  return (uint32_t)f2bf(silu_mul_f32(g0, u0)) | ((uint32_t)f2bf(silu_mul_f32(g1, u1)) << 16);
}

// eight packed bf16 of gate and up -> eight packed bf16 products
__device__ __forceinline__ uint4 silu_mul8(const uint4 g, const uint4 u) {
  return make_uint4(silu_mul_pair(g.x, u.x), silu_mul_pair(g.y, u.y), silu_mul_pair(g.z, u.z), silu_mul_pair(g.w, u.w));
}

}  // namespace agq
