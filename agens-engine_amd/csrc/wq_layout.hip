// Load-time repack (int4 container -> W4 / W3 / W2 KT) and dequant (KT -> dense bf16 rows) for gfx950.
//
// The KT byte layout is the reference's (kernels/src/w4_gemv.cu:13-31, :439-458, :758-790) so weights repacked here
// are interchangeable with the reference's; the kernels are written for wave64: one thread per 16-byte lane chunk of
// the output, consecutive threads writing consecutive chunks of a record (fully coalesced stores), grid-stride loops.
#include <map>
#include <vector>
#include <mutex>
#include <utility>

#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {

// compute units of the current device (cached)
int num_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
  }
  return cus;
}

// Library scratch per (device, stream), as the reference keeps its split-K partials and counters
// (w4_gemv.cu:2096-2118): allocated zero-filled on first use and grown (at least doubling) when a launch needs more,
// never inside a stream capture (null then: the caller takes a path without scratch).  Every buffer handed out is held
// until the process ends, the replaced ones included, so launches still in flight and graphs captured before a growth
// keep valid memory.  Launches on one stream are ordered, so they share it safely.  Users keep their counters (the
// first 4 KB) at zero between launches.
//
// A caller that must not allocate (ak_wq_gemv_kt_multi_noalloc) installs a fixed buffer for the calling thread first:
// then this returns that buffer when it is large enough and null otherwise, and never allocates.
ScratchOverride& scratch_override() {
  static thread_local ScratchOverride o;
  return o;
}

void* stream_scratch(hipStream_t s, size_t bytes) {
  const ScratchOverride& o = scratch_override();
  if (o.on) return bytes <= o.bytes ? o.p : nullptr;
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> bufs;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  auto& b = bufs[{dev, s}];
  if (b.first && b.second >= bytes) return b.first;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;
  }
  // at least double: a replaced buffer is kept, not freed (a graph captured before the growth still addresses it), so
  // the retired buffers stay below the current one in total
  size_t want = bytes > ((size_t)4 << 20) ? bytes : ((size_t)4 << 20);
  if (b.first && want < 2 * b.second) want = 2 * b.second;
  void* p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess || hipMemset(p, 0, want) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    if (p) (void)hipFree(p);
    (void)hipGetLastError();
    return nullptr;
  }
  static std::vector<void*> retired;
  if (b.first) retired.push_back(b.first);
  b = {p, want};
  return p;
}

namespace {

// Morton-style bit spreading: 8 two-bit fields (low 16 bits) -> the low 2 bits of 8 nibbles; 8 bits -> bit 0 of 8
// nibbles.  Used to expand W3 / W2 lane chunks back to W4 nibble words.
__device__ __forceinline__ uint32_t spread_2to4(uint32_t v) {
  v &= 0xFFFFu;
  v = (v ^ (v << 8)) & 0x00FF00FFu;
  v = (v ^ (v << 4)) & 0x0F0F0F0Fu;
  v = (v ^ (v << 2)) & 0x33333333u;
  return v;
}
__device__ __forceinline__ uint32_t spread_1to4(uint32_t v) {
  v &= 0xFFu;
  v = (v ^ (v << 12)) & 0x000F000Fu;
  v = (v ^ (v << 6)) & 0x03030303u;
  v = (v ^ (v << 3)) & 0x11111111u;
  return v;
}

// lane chunk `c` of record `rec` as 4 W4 nibble words (nibble = q + 8)
template <int BITS>
__device__ __forceinline__ uint4 chunk_nibbles(const void* wt, size_t rec, int c) {
  if (BITS == 4) return reinterpret_cast<const uint4*>(wt)[rec * 32 + c];
  const uint32_t* r = reinterpret_cast<const uint32_t*>(wt) + rec * (32 * BITS);
  const uint2 lo = reinterpret_cast<const uint2*>(r)[c];
  if (BITS == 2)
    return make_uint4(spread_2to4(lo.x) + 0x66666666u, spread_2to4(lo.x >> 16) + 0x66666666u,
                      spread_2to4(lo.y) + 0x66666666u, spread_2to4(lo.y >> 16) + 0x66666666u);
  const uint32_t h = r[64 + c];
  return make_uint4((spread_2to4(lo.x) | (spread_1to4(h) << 2)) + 0x44444444u,
                    (spread_2to4(lo.x >> 16) | (spread_1to4(h >> 8) << 2)) + 0x44444444u,
                    (spread_2to4(lo.y) | (spread_1to4(h >> 16) << 2)) + 0x44444444u,
                    (spread_2to4(lo.y >> 16) | (spread_1to4(h >> 24) << 2)) + 0x44444444u);
}

// container -> KT.  Thread = one lane chunk (32 inputs) of one record; scales copied by the first chunk of each
// group.  W3 / W2: n = nibble - (8 - 2^(BITS-1)) must lie in [0, 2^BITS); a violation sets *bad (the chunk is still
// written with the value masked, as the reference does).
template <int BITS, int G>
__global__ void __launch_bounds__(256) repack_kernel(const uint4* __restrict__ src, const uint16_t* __restrict__ ssrc,
                                                     void* __restrict__ dst, uint16_t* __restrict__ sdst, int n, int k,
                                                     int* __restrict__ bad) {
  constexpr int SPT = 1024 / G, CPG = G / 32;
  constexpr int OFF = 8 - (1 << (BITS - 1)), MAXN = (1 << BITS) - 1;
  const int chunks = k >> 5, groups = k / G, tiles = kpad(k) >> 10;
  const size_t total = (size_t)tiles * n * 32;
  int my_bad = 0;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(i & 31);
    const size_t rec = i >> 5;
    const int o = (int)(rec % (size_t)n), t = (int)(rec / (size_t)n);
    const int cg = t * 32 + c;
    const uint4 q = cg < chunks ? src[(size_t)o * chunks + cg] : make_uint4(0x88888888u, 0x88888888u, 0x88888888u,
                                                                             0x88888888u);
    if (BITS == 4) {
      reinterpret_cast<uint4*>(dst)[i] = q;
    } else {
      const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
      uint32_t lo[2] = {0u, 0u}, hi = 0u;
#pragma unroll
      for (int v = 0; v < 32; ++v) {
        const int nv = (int)((qw[v >> 3] >> (4 * (v & 7))) & 0xFu) - OFF;
        my_bad |= (nv < 0) | (nv > MAXN);
        const uint32_t mv = (uint32_t)nv & (uint32_t)MAXN;
        lo[v >> 4] |= (mv & 3u) << (2 * (v & 15));
        if (BITS == 3) hi |= (mv >> 2) << v;
      }
      uint32_t* r = reinterpret_cast<uint32_t*>(dst) + rec * (32 * BITS);
      reinterpret_cast<uint2*>(r)[c] = make_uint2(lo[0], lo[1]);
      if (BITS == 3) r[64 + c] = hi;
    }
    if (c % CPG == 0) {
      const int g = cg / CPG;
      sdst[rec * SPT + c / CPG] = g < groups ? ssrc[(size_t)o * groups + g] : (uint16_t)0;
    }
  }
  if (BITS != 4 && my_bad) atomicOr(bad, 1);
}

// KT rows [r0, r0 + nr) -> dense bf16 w [nr][k], w = bf16_rn(q * scale) (the product is exact in fp32; the conversion
// rounds to nearest even).  Thread = 8 consecutive outputs of a row (16 bytes): consecutive threads write consecutive
// 16-byte pieces of a row and read consecutive words of its KT record (per lane chunk of 32 inputs: W4 4 words of
// nibbles; W2 2 words of 2-bit codes; W3 those and a word of third bits, one byte per 8 inputs).
template <int BITS, int G>
__global__ void __launch_bounds__(256) dequant_kernel(const void* __restrict__ wt, const uint16_t* __restrict__ st,
                                                      uint16_t* __restrict__ w, int n, int k, int r0, int nr) {
  constexpr int SPT = 1024 / G, CPG = G / 32;
  const int kw = k >> 3;  // 16-byte pieces per output row
  const size_t total = (size_t)nr * kw;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int o = (int)(i / (size_t)kw), e = (int)(i - (size_t)o * kw);
    const int t = e >> 7, c = (e >> 2) & 31, u = e & 3;  // 1024-input tile, lane chunk, word of the chunk
    const size_t rec = (size_t)t * n + r0 + o;
    const uint32_t* r = reinterpret_cast<const uint32_t*>(wt) + rec * (32 * BITS);
    uint32_t q;  // 8 nibbles, value = nibble - 8
    if constexpr (BITS == 4) {
      q = r[c * 4 + u];
    } else {
      const uint32_t lo = spread_2to4(r[c * 2 + (u >> 1)] >> (16 * (u & 1)));
      if constexpr (BITS == 2) q = lo + 0x66666666u;
      else q = (lo | (spread_1to4(r[64 + c] >> (8 * u)) << 2)) + 0x44444444u;
    }
    const float s = bf2f(st[rec * SPT + c / CPG]), m8 = -8.0f * s;
    const uint32_t ev = q & 0x0F0F0F0Fu, od = (q >> 4) & 0x0F0F0F0Fu;  // inputs 2b, 2b + 1 in byte b
    uint32_t v[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      const bf16x2 p = {(__bf16)fmaf((float)((ev >> (8 * b)) & 0xFFu), s, m8),
                        (__bf16)fmaf((float)((od >> (8 * b)) & 0xFFu), s, m8)};
      v[b] = __builtin_bit_cast(uint32_t, p);
    }
    reinterpret_cast<uint4*>(w + (size_t)o * k)[e] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

bool group_ok(int k, int group) { return (group == 64 || group == 128) && k % group == 0; }

template <int BITS>
int launch_repack(const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, int group, int* bad,
                  hipStream_t s) {
  const size_t total = (size_t)(kpad(k) >> 10) * n * 32;
  const int blocks = (int)((total + 255) / 256 < (size_t)num_cus() * 16 ? (total + 255) / 256 : (size_t)num_cus() * 16);
  auto kern = group == 64 ? repack_kernel<BITS, 64> : repack_kernel<BITS, 128>;
  hipLaunchKernelGGL(kern, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, s, reinterpret_cast<const uint4*>(packed),
                     static_cast<const uint16_t*>(scales), wt, static_cast<uint16_t*>(st), n, k, bad);
  return (int)hipGetLastError();
}

}  // namespace
}  // namespace agq

using namespace agq;

extern "C" {

size_t ak_w4_kt_weight_bytes(int n, int k) { return (size_t)n * kpad(k) / 2; }
size_t ak_w4_kt_scale_bytes(int n, int k, int group) { return (size_t)n * kpad(k) / group * 2; }
size_t ak_w4g128_kt_weight_bytes(int n, int k) { return ak_w4_kt_weight_bytes(n, k); }
size_t ak_w4g128_kt_scale_bytes(int n, int k) { return ak_w4_kt_scale_bytes(n, k, 128); }
size_t ak_wq_kt_weight_bytes(int bits, int n, int k) { return (size_t)n * kpad(k) * bits / 8; }
size_t ak_w3_kt_weight_bytes(int n, int k) { return ak_wq_kt_weight_bytes(3, n, k); }

int ak_w4_repack_kt(const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, int group,
                    void* stream) {
  if (!group_ok(k, group) || k % 32 != 0 || n < 1) return AK_INVALID;
  return launch_repack<4>(packed, scales, wt, st, n, k, group, nullptr, static_cast<hipStream_t>(stream));
}

int ak_w4g128_repack_kt(const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, void* stream) {
  return ak_w4_repack_kt(packed, scales, wt, st, n, k, 128, stream);
}

// W3 / W2: the range flag is read back, so this call synchronizes `stream` (load time only).
int ak_wq_repack_kt(int bits, const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, int group,
                    void* stream) {
  if (bits == 4) return ak_w4_repack_kt(packed, scales, wt, st, n, k, group, stream);
  if ((bits != 2 && bits != 3) || !group_ok(k, group) || k % 32 != 0 || n < 1) return AK_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int* bad = nullptr;
  if (hipMalloc(&bad, sizeof(int)) != hipSuccess) return AK_OOM;
  int e = (int)hipMemsetAsync(bad, 0, sizeof(int), s);
  if (!e)
    e = bits == 3 ? launch_repack<3>(packed, scales, wt, st, n, k, group, bad, s)
                  : launch_repack<2>(packed, scales, wt, st, n, k, group, bad, s);
  int h = 0;
  if (!e) e = (int)hipMemcpyAsync(&h, bad, sizeof(int), hipMemcpyDeviceToHost, s);
  if (!e) e = (int)hipStreamSynchronize(s);
  (void)hipFree(bad);
  if (e) return e;
  return h ? AK_INVALID : 0;
}

int ak_w3_repack_kt(const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, int group,
                    void* stream) {
  return ak_wq_repack_kt(3, packed, scales, wt, st, n, k, group, stream);
}

int ak_wq_dequant_kt_rows(int bits, const void* wt, const void* st, void* w, int n, int k, int group, int r0, int nr,
                          void* stream) {
  if (!group_ok(k, group) || k % 32 != 0 || r0 < 0 || nr < 1 || r0 + nr > n) return AK_INVALID;
  decltype(&dequant_kernel<4, 128>) kern;
  switch (bits * 1000 + group) {
    case 4128: kern = dequant_kernel<4, 128>; break;
    case 4064: kern = dequant_kernel<4, 64>; break;
    case 3128: kern = dequant_kernel<3, 128>; break;
    case 3064: kern = dequant_kernel<3, 64>; break;
    case 2128: kern = dequant_kernel<2, 128>; break;
    case 2064: kern = dequant_kernel<2, 64>; break;
    default: return AK_INVALID;
  }
  const size_t total = (size_t)nr * (k >> 3);
  const size_t want = (total + 255) / 256, cap = (size_t)num_cus() * 16;
  hipLaunchKernelGGL(kern, dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     wt, static_cast<const uint16_t*>(st), static_cast<uint16_t*>(w), n, k, r0, nr);
  return (int)hipGetLastError();
}

int ak_w4_dequant_kt(const void* wt, const void* st, void* w, int n, int k, int group, void* stream) {
  return ak_wq_dequant_kt_rows(4, wt, st, w, n, k, group, 0, n, stream);
}
int ak_w4_dequant_kt_rows(const void* wt, const void* st, void* w, int n, int k, int group, int r0, int nr,
                          void* stream) {
  return ak_wq_dequant_kt_rows(4, wt, st, w, n, k, group, r0, nr, stream);
}
int ak_w3_dequant_kt_rows(const void* wt, const void* st, void* w, int n, int k, int group, int r0, int nr,
                          void* stream) {
  return ak_wq_dequant_kt_rows(3, wt, st, w, n, k, group, r0, nr, stream);
}

}  // extern "C"
