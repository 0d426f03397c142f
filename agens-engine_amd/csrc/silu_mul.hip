// SiLU(gate) * up over the merged gate_up output (the activation between the gate_up and down projections), gfx950.
// Reference: ak_silu_mul / ak_silu_mul_part, kernels/src/fastmath/silu_mul.cu:10-72: out[t][i] =
// bf16(g / (1 + exp(-g)) * u), g = gate_up[t][i], u = gate_up[t][inter + i] (bf16 in, fp32 math, one bf16 rounding).
// The reference compiles that expression with CUDA's fast-math approximations of exp and of the division; here exp is
// the device library's expf and the division an fp32 division, so results agree with the reference within the
// approximations' error (at most one bf16 unit in the last place of the rounded result), not bit for bit.
// silu_mul_f32 is the one definition of the value: the GEMV kernels that apply it to their activations as they load
// them (the down projection of a decoder layer) use the same function, so fused and separate results are identical.
#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_silu.h"

namespace agq {
namespace {

// tokens x inter / 8 vectors of 8 outputs
__global__ void silu_mul_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, unsigned nv, unsigned total) {
  const unsigned tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= total) return;
  const unsigned t = tid / nv, off = tid - t * nv;
  out[tid] = silu_mul8(in[(size_t)t * nv * 2 + off], in[(size_t)t * nv * 2 + nv + off]);
}

// one tensor-parallel share [gate share | up share] (np each) -> the full row of inter with the share's products at
// [lo, lo + np) and zeros elsewhere
__global__ void silu_mul_part_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, unsigned inter8, unsigned lo8,
                                     unsigned np8) {
  const unsigned tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= inter8) return;
  if (tid < lo8 || tid >= lo8 + np8) {
    out[tid] = make_uint4(0u, 0u, 0u, 0u);
    return;
  }
  const unsigned off = tid - lo8;
  out[tid] = silu_mul8(in[off], in[np8 + off]);
}

}  // namespace
}  // namespace agq

extern "C" int ak_silu_mul(const void* gate_up, void* out, int tokens, int inter, void* stream) {
  // the reference's check (silu_mul.cu:67), and null pointers / negative sizes
  if (!gate_up || !out || tokens < 0 || inter < 0 || inter % 8) return AK_INVALID;
  const unsigned nv = (unsigned)inter / 8, total = nv * (unsigned)tokens;
  if (!total) return 0;
  hipLaunchKernelGGL(agq::silu_mul_kernel, dim3((total + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(gate_up), static_cast<uint4*>(out), nv, total);
  return (int)hipGetLastError();
}

extern "C" int ak_silu_mul_part(const void* gate_up_part, void* out, int inter, int lo, int np, void* stream) {
  // the reference's checks (silu_mul.cu:59)
  if (!gate_up_part || !out || inter < 0 || lo < 0 || np < 0 || inter % 8 || lo % 8 || np % 8 || lo + np > inter)
    return AK_INVALID;
  const unsigned n8 = (unsigned)inter / 8;
  if (!n8) return 0;
  hipLaunchKernelGGL(agq::silu_mul_part_kernel, dim3((n8 + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(gate_up_part), static_cast<uint4*>(out), n8, (unsigned)lo / 8,
                     (unsigned)np / 8);
  return (int)hipGetLastError();
}
