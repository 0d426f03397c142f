// SiLU(gate) * up over the merged gate_up output (the activation between the gate_up and down projections), gfx950.
// Reference entry points: ak_silu_mul / ak_silu_mul_part, kernels/src/fastmath/silu_mul.cu:10-72: out[t][i] =
// bf16(g / (1 + exp(-g)) * u), g = gate_up[t][i], u = gate_up[t][inter + i] (bf16 in, fp32 math, one bf16 rounding).
// The reference compiles that expression with CUDA's fast-math approximations of exp and of the division; here exp is
// the device library's expf and the division an fp32 division, so results agree with the reference within the
// approximations' error (at most one bf16 unit in the last place of the rounded result), not bit for bit.
// silu_mul8 (wq_silu.h) is the one definition of the value: the GEMV kernels that apply it to their activations as they
// load them (the down projection of a decoder layer) use the same function, so fused and separate results are
// identical.
//
// One kernel serves both entry points.  An output row of `cols` 16-byte vectors (8 bf16 each) has a window
// [win_lo, win_lo + win_n) of vectors that are products; the vectors outside it are zeros.  Window vector j of row r
// takes its gate from source vector src_row * r + j and its up value win_n vectors further on:
//   ak_silu_mul:       window = the whole row, source rows [gate | up] of 2 * cols vectors;
//   ak_silu_mul_part:  one row, window = the share [lo, lo + np), source = [gate share | up share].
// The grid strides over rows in y and over a row's vectors in x (wave64 workgroups of 256 threads, at most 1024 of
// them per row, each thread 16-byte loads and stores), so any row length runs with a bounded grid.
#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_silu.h"

namespace agq {
namespace {

constexpr int kSiluThreads = 256;
constexpr unsigned kSiluMaxGridX = 1024, kSiluMaxGridY = 65535;

struct SiluRows {
  const uint4* src;
  uint4* dst;
  unsigned cols;     // vectors per output row
  unsigned win_lo;   // first product vector of a row
  unsigned win_n;    // product vectors per row (the gate -> up distance in the source, in vectors)
  size_t src_row;    // source vectors per row
};

__global__ void __launch_bounds__(kSiluThreads) silu_rows_kernel(const SiluRows a, unsigned rows) {
  for (size_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const uint4* const gate = a.src + r * a.src_row;
    uint4* const out = a.dst + r * a.cols;
    for (unsigned v = blockIdx.x * kSiluThreads + threadIdx.x; v < a.cols; v += gridDim.x * kSiluThreads) {
      const unsigned j = v - a.win_lo;  // wraps past the window's end when v < win_lo
      out[v] = j < a.win_n ? silu_mul8(gate[j], gate[a.win_n + j]) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

int launch_silu_rows(const SiluRows& a, unsigned rows, hipStream_t s) {
  if (!rows || !a.cols) return 0;
  const unsigned gy = rows < kSiluMaxGridY ? rows : kSiluMaxGridY;  // rows beyond it: the y stride
  unsigned gx = (a.cols + kSiluThreads - 1) / kSiluThreads;
  gx = gx < kSiluMaxGridX ? gx : kSiluMaxGridX;
  hipLaunchKernelGGL(silu_rows_kernel, dim3(gx, gy), dim3(kSiluThreads), 0, s, a, rows);
  return (int)hipGetLastError();
}

}  // namespace
}  // namespace agq

// reference: silu_mul.cu:66-72 (inter % 8 == 0, else 1); null pointers and negative sizes are refused too
extern "C" int ak_silu_mul(const void* gate_up, void* out, int tokens, int inter, void* stream) {
  if (!gate_up || !out || tokens < 0 || inter < 0 || inter % 8) return AK_INVALID;
  agq::SiluRows a;
  a.src = static_cast<const uint4*>(gate_up);
  a.dst = static_cast<uint4*>(out);
  a.cols = (unsigned)inter / 8;
  a.win_lo = 0;
  a.win_n = a.cols;
  a.src_row = 2 * (size_t)a.cols;
  return agq::launch_silu_rows(a, (unsigned)tokens, static_cast<hipStream_t>(stream));
}

// reference: silu_mul.cu:58-64 (inter, lo, np multiples of 8 and lo + np <= inter, else 1)
extern "C" int ak_silu_mul_part(const void* gate_up_part, void* out, int inter, int lo, int np, void* stream) {
  if (!gate_up_part || !out || inter < 0 || lo < 0 || np < 0 || inter % 8 || lo % 8 || np % 8 || lo + np > inter)
    return AK_INVALID;
  agq::SiluRows a;
  a.src = static_cast<const uint4*>(gate_up_part);
  a.dst = static_cast<uint4*>(out);
  a.cols = (unsigned)inter / 8;
  a.win_lo = (unsigned)lo / 8;
  a.win_n = (unsigned)np / 8;
  a.src_row = 0;
  return agq::launch_silu_rows(a, 1u, static_cast<hipStream_t>(stream));
}
