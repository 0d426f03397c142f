// Shared definitions of the MI355X (gfx950) mixed-bit group-quantized GEMV library.
//
// Weight layout (unchanged from the reference, kernels/src/w4_gemv.cu:13-31): k is padded to kp = ceil(k/1024)*1024
// and split into tiles of 1024 inputs; tile t of output row o is one contiguous record at (t * n + o) * 128 * BITS
// bytes.  Inside a record, "lane chunk" c (0..31) covers inputs 32c .. 32c+31 of the tile:
//   W4: bytes 16c .. 16c+15 = 4 words of 8 nibbles (nibble = q + 8, low nibble = lowest input);
//   W3: words 2c, 2c+1 = 2-bit low fields of inputs 0-15 / 16-31 (field at bit 2*(i%16)), word 64+c bit i = bit 2 of
//       input i; value n = q + 4;
//   W2: words 2c, 2c+1 = 2-bit fields, value n = q + 2.
// Scales: bf16 at (t * n + o) * (1024 / G) + slot, one per group of G inputs (G = 64 or 128).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace agq {

constexpr int kMaxSegs = 4;

// Up to 4 linears that share x, k, group and bits in one launch.  Rows of segment i occupy global rows
// [end[i-1], end[i-1] + n[i]) of a concatenated row space in which every segment is padded to a multiple of `pad`
// rows (end[] are the cumulative padded ends).  Token j of segment i is written at y[i] + j * ldy[i].
struct Segs {
  const void* wt[kMaxSegs];
  const uint16_t* st[kMaxSegs];
  uint16_t* y[kMaxSegs];
  int n[kMaxSegs];
  int end[kMaxSegs];
  int ldy[kMaxSegs];
  int nseg;
};

__host__ __device__ inline int kpad(int k) { return (k + 1023) & ~1023; }

// A fixed scratch buffer that replaces the per-stream library scratch for the calling host thread while `on` (the
// entry point that allocates nothing installs it around its launches).
struct ScratchOverride {
  void* p = nullptr;
  size_t bytes = 0;
  bool on = false;
};
ScratchOverride& scratch_override();

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// streaming 16-byte load (weights are read exactly once per launch: nontemporal hint)
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_stream2(const uint2* p) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld_stream1(const uint32_t* p) { return __builtin_nontemporal_load(p); }

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// segment of a global (padded, concatenated) row
__device__ __forceinline__ int seg_of(const Segs& s, int grow) {
  int sg = 0;
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) sg += (i < s.nseg && grow >= s.end[i - 1]) ? 1 : 0;
  return sg;
}

}  // namespace agq

// hipError_t values the reference's callers test for (crates/agens-cuda/src/lib.rs:49-55, :187-190)
#define AK_INVALID ((int)hipErrorInvalidValue)
#define AK_OOM ((int)hipErrorOutOfMemory)
