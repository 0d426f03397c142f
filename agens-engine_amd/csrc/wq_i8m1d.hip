// The default-numerics GEMV for up to 8 tokens (decode and small M), group 128, on gfx950: the same exact integer
// group sums and the same fp32 combine order as wq_i8.hip (rows are bit-identical to any-m launches), with an MFMA
// layout chosen so that every weight load instruction reads whole cache lines.
//
// "Diagonal" layout of v_mfma_i32_16x16x64_i8 for a block of 4 output rows and one quad (4 groups = 16 lane chunks):
//   lane (c, h) = (lane % 16, lane / 16);
//   B column c = (row c >> 2 of the block, group c & 3 of the quad): lane (c, h) holds chunk 4 * (c & 3) + h of that
//     row;
//   A row c = (group c >> 2, limb c & 3): lane (c, h) holds limb c & 3 of the inputs of chunk 4 * (c >> 2) + h
//     (limb 3 is zero);
//   D[4g + j][4r + v] is the limb-j sum of row r with the inputs of group g; only g == v is used ("the diagonal"):
//     lane (c, h) with (c & 3) == h holds group h of row c >> 2 in its accumulators (limbs 0..2).
// The MFMA work per weight is the same as a 16-row layout (13 of 16 A rows or columns are wasted either way), but the
// A operand has 12 useful rows instead of 3, and row blocks are 4 rows, so work divides evenly over 256 CUs.
//
// Items are tiles: 4 rows x one 1024-input tile (two quads), the whole of those rows' tile records, so every load
// instruction covers whole 128-byte lines at once (a quad of a W3 record is half of each of its lines, and loads
// of half lines reach about 4.4 TB/s against 6.5 for whole ones).  W4: one 16-byte load per quad (4 rows x 256 B).
// W2 and the W3 two-bit planes: one 16-byte load covers both quads: lane (c, h) reads the chunk pair {2 (h >> 1),
// 2 (h >> 1) + 1} of group (c & 3) + 4 (h & 1); one v_permlane16_swap per dword pair (odd 16-lane rows of the first
// operand <-> even rows of the second) then leaves the quad-0 diagonal operand in the first and the quad-1 operand
// in the second.  The W3 third-bit plane: one 8-byte load of the same chunk pair, swapped the same way.
//
// Work decomposition: one persistent workgroup per CU owns a contiguous range of 4-row blocks of one segment.  Its
// tasks are (block, stripe set j < SPLIT) pairs: stripe set j = the contiguous stripes [j P / SPLIT, (j + 1) P / SPLIT),
// i.e. a contiguous run of tiles, walked in order (the fp32 order of the numerics).  Wave w always takes stripe set
// w % SPLIT, for the blocks w / SPLIT, w / SPLIT + nwv / SPLIT, ...  With SPLIT = 1 a wave owns whole blocks and adds
// the stripe partials itself; otherwise the partials meet in LDS and the last task of a block to finish (LDS ticket)
// adds them in stripe order.
//
// Item pipeline: every wave streams its items through DEPTH register buffers.  A group of DEPTH items is one
// branch-free block of code, so the compiler interleaves the unpacking, LDS reads and MFMAs of neighbouring items:
// the load offsets are a fixed per-lane part plus a scalar part of (block, tile), the cursors advance by selects,
// and a stripe that ends inside the group only leaves a copy of its accumulators; the group's epilogue turns those
// into stripe partials.
#include <atomic>
#include <stdlib.h>

#include <vector>

#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_i8_common.h"

// tile items in flight per wave (register buffers) for one or two tokens
#ifndef AK_M1_TILES
#define AK_M1_TILES 2
#endif

namespace agq {

int num_cus();
void* stream_scratch(hipStream_t s, size_t bytes);

namespace {

constexpr int kG = 128, kCPQ = 16;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, dword 3 (CDNA)
constexpr int kNt = 2;                    // streaming (non-temporal) cache policy for the weights
constexpr int kVmcnt0 = 0x0F70;            // s_waitcnt immediate: vector memory counter 0, the others unconstrained
constexpr int kSc1 = 16;                  // device-scope coherent access (sc1): misses / writes through the L2

// one tile item of one lane: the raw weight words of both quads (before the W2 / W3 lane exchange) and the dwords
// holding the two quads' scales
template <int BITS>
struct TileRaw;
template <>
struct TileRaw<4> { uint4 q0, q1; uint32_t s0, s1; };
template <>
struct TileRaw<3> { uint4 lo; uint2 hi; uint32_t s0, s1; };
template <>
struct TileRaw<2> { uint4 lo; uint32_t s0, s1; };

// v_permlane16_swap: .x = a with its odd 16-lane rows replaced by the even rows of b, .y = b with its even rows
// replaced by the odd rows of a
__device__ __forceinline__ uint2 swap16(uint32_t a, uint32_t b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  return make_uint2(r[0], r[1]);
}

// the per-quad raw operands of a tile item (quad 0 -> r0, quad 1 -> r1)
template <int BITS>
__device__ __forceinline__ void split_tile(const TileRaw<BITS>& t, Raw<BITS>& r0, Raw<BITS>& r1) {
  if constexpr (BITS == 4) {
    r0.w = t.q0;
    r1.w = t.q1;
  } else {
    const uint2 a = swap16(t.lo.x, t.lo.z), b = swap16(t.lo.y, t.lo.w);
    r0.lo = make_uint2(a.x, b.x);
    r1.lo = make_uint2(a.y, b.y);
    if constexpr (BITS == 3) {
      const uint2 hh = swap16(t.hi.x, t.hi.y);
      r0.hi = hh.x;
      r1.hi = hh.y;
    }
  }
}

// segment field i (i < 4, wave-uniform) by constant-index selects: indexing the kernel-argument arrays dynamically
// makes the compiler hold their address in vector registers
template <typename T>
__device__ __forceinline__ T pick4(int i, T v0, T v1, T v2, T v3) {
  return i == 0 ? v0 : i == 1 ? v1 : i == 2 ? v2 : v3;
}
#define AK_PICK(i, arr) pick4((i), (arr)[0], (arr)[1], (arr)[2], (arr)[3])
static_assert(kMaxSegs == 4, "segment selects cover four segments");

// Chained launches (several GEMV steps in one persistent launch): a workgroup signals the end of a step by writing
// its flag word (one per workgroup, 64 bytes apart) with the step count, after its outputs are stored with
// device-coherent (sc1, L2 write-through) stores and acknowledged; a step that reads earlier steps' outputs first
// issues its first weight loads (constant data), then waits until every workgroup's flag has reached the step, then
// reads its activations with device-coherent loads.  No L2 write-back or invalidate is needed on either side.
// Flags are packed 4 bytes apart (AK_CHAIN_DENSE, the default): a poll reads 16 flags per 64-byte line, one 16-byte
// load per lane, so a poll round of the whole GPU is 256 x 16 line requests instead of 256 x 256 (each one a miss
// of the L2, since the loads are device-coherent).
#ifndef AK_CHAIN_DENSE
#define AK_CHAIN_DENSE 1
#endif
constexpr int kChainMaxWg = 1024, kChainFlagStride = AK_CHAIN_DENSE ? 1 : 16;
constexpr long long kChainSpinTicks = 20000000;  // 0.2 s of the 100 MHz wall clock: a bounded wait, then an error
__device__ __attribute__((aligned(256))) uint32_t g_chain_flags[kChainMaxWg * kChainFlagStride];
__device__ uint32_t g_chain_err;

// Tagged activations: where a step's x is the output of the step just before it, that step also writes its outputs
// as 32-bit words (bf16 value | tag << 16, tag = the low 16 bits of the chain's launch count + 1) to a buffer of the
// chain, and the step reads that buffer instead of waiting at the grid barrier: each wave reads its own activations
// (first through the L2, then device-coherently) until every word it holds carries the launch's tag.  One
// write-through and one read round trip then separate the steps, instead of the write acknowledgement, the flag
// store, the poll and the activation read of the barrier.
// x complete means every workgroup of the step before has finished it (outputs are written at the end of a step, and
// every output row is written); the host takes a tagged wait only where that step itself waited for the one before
// it and the step after this one waits, so that the grid-barrier guarantee (every earlier step complete) still holds
// wherever a later step relies on it.
constexpr uint32_t kTagMask = 0xFFFFu;
// the first read of a step's tagged activations goes through the L2 (1) or device-coherently (0)
#ifndef AK_TAG_CACHED_FIRST
#define AK_TAG_CACHED_FIRST 1
#endif
// weight items of a tagged step requested before its activations are waited for (measured at M = 1: 1 of the 2 in
// flight about 0.4 % faster than 2, none 1.5 % slower)
#ifndef AK_TAG_PREFETCH
#define AK_TAG_PREFETCH 1
#endif


// Wave 0 polls until the flags of workgroups [0, nwg) are all at least `target` (wrap-safe).  It polls before it
// requests weights of its own, so that no poll waits behind them.
__device__ __forceinline__ void chain_poll(uint32_t target) {
  const int lane = threadIdx.x, nwg = gridDim.x;
  const long long t0 = wall_clock64();
  for (;;) {
    bool ok = true;
    if constexpr (AK_CHAIN_DENSE) {
      const __amdgpu_buffer_rsrc_t rf =
          __builtin_amdgcn_make_buffer_rsrc(g_chain_flags, (short)0, kChainMaxWg * 4, kRsrcWord3);
      for (int j = 4 * lane; j < nwg; j += 256) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rf, j * 4, 0, kSc1);
#pragma unroll
        for (int i = 0; i < 4; ++i) ok = ok && (j + i >= nwg || (int)(v[i] - target) >= 0);
      }
    } else {
      for (int j = lane; j < nwg; j += 64) {
        const uint32_t v = __hip_atomic_load(g_chain_flags + j * kChainFlagStride, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        ok = ok && (int)(v - target) >= 0;
      }
    }
    if (__all(ok)) break;
    if (wall_clock64() - t0 > kChainSpinTicks) {
      if (lane == 0) __hip_atomic_store(&g_chain_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// the workgroup meets at an LDS-only barrier (the weight loads in flight stay in flight)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One GEMV step of one workgroup.  CHAIN: part of a chained launch (workgroups past the step's grid return at once;
// with `wait`, the step waits for all workgroups to reach `target` after its first weight requests; with a.xtg, it
// polls its tagged activations for `tag` instead; activations are read and outputs written device-coherently, and
// the tagged copy of the outputs is written where a.ytg asks for it).
//
// SK (split-K across workgroups, one segment): workgroup (r, p) computes stripe p of the rows of range r, converting
// only that stripe's activations; it writes its stripe partials with device-coherent stores, and the last of the
// range's P workgroups (device-scope counter) adds them in stripe order and writes y.
template <int BITS, int SPLIT, int DEPTH, int MT, bool CHAIN, bool SK = false, bool ACT = false>
__device__ __forceinline__ void m1d_body(const I8Args& a, uint8_t* lds, bool wait, uint32_t target, uint32_t tag) {
  static_assert(!SK || SPLIT == 1, "a split launch gives every wave whole stripes of its blocks");
  constexpr int LPU = kG / 8, UPW = 64 / LPU, XB = 4;
  constexpr int REC = 128 * BITS;  // one row's tile record
  const int P = a.P, nquad = a.nquad, k = a.k, mm = a.m;  // mm <= MT tokens (the others are zero, not written)
  const int ntile = nquad >> 1;
  const int nwv = CHAIN ? 16 : blockDim.x >> 6;  // a chained launch has 16 waves
  const int lg_nwv = CHAIN ? 4 : __builtin_ctz((unsigned)nwv);  // 8 or 16 waves: divisions by shifts
  int tid = threadIdx.x;
  // chained: an opaque thread index per step, so that nothing lane-dependent is hoisted out of the step loop (the
  // hoisted values would stay live across every step's item loop)
  if constexpr (CHAIN) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int rr = c >> 2, vv = c & 3;  // B role: row of the block, group of the quad
  const Segs& sgs = a.segs;

  // no rows of this step: the workgroup still passes the step's wait (wave 0 polls; the chain's barrier after the step
  // holds the other waves), so that a later step declared independent never reads what the steps before this one
  // write before they have written it
  if (CHAIN && (int)blockIdx.x >= AK_PICK(sgs.nseg - 1, a.wg_end)) {
    if (wait && (threadIdx.x >> 6) == 0) chain_poll(target);
    return;
  }
  // this workgroup's segment and its blocks [b_lo, b_lo + nb) of that segment (SK: row range r, stripe psk; the
  // ranges are wg_end[0] / P)
  int sg = 0;
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) sg += (i < sgs.nseg && (int)blockIdx.x >= a.wg_end[i - 1]) ? 1 : 0;
  const int nr = SK ? div_by_p(a.wg_end[0], a) : 1, r = SK ? div_by_p((int)blockIdx.x, a) : 0;
  const int psk = SK ? (int)blockIdx.x - r * P : 0;
  // first tile of stripe p (the launch's multiplier: no scalar branches on P)
  auto stripe_tile = [&](int p) { return div_by_p(p * ntile, a); };
  const int wg0 = sg ? AK_PICK(sg - 1, a.wg_end) : 0, gs = SK ? nr : AK_PICK(sg, a.wg_end) - wg0;
  const int w = SK ? r : (int)blockIdx.x - wg0;
  const int n = AK_PICK(sg, sgs.n), n_b4 = (n + 3) >> 2;
  // the quads the activation image holds: [q0, q0 + nqs) (SK: stripe psk; else all)
  const int q0 = SK ? 2 * stripe_tile(psk) : 0;
  const int nqs = SK ? 2 * stripe_tile(psk + 1) - q0 : nquad;
  // 32-bit divisions (w < 1024 workgroups, < 2^21 blocks): a 64-bit one is a long instruction sequence on the GPU
  const int b_lo = (int)((unsigned)w * (unsigned)n_b4 / (unsigned)gs);
  const int nb = (int)((unsigned)(w + 1) * (unsigned)n_b4 / (unsigned)gs) - b_lo;
  uint16_t* const yseg = AK_PICK(sg, sgs.y);
  uint32_t* const ytg = CHAIN ? AK_PICK(sg, a.ytg) : nullptr;
  const int ldy = AK_PICK(sg, sgs.ldy);

  // LDS: zeros [512 B] | limbs [MT][nquad][half 2][chunk 16][limb 3][16 B] | meta [MT][nquad][4] int4 |
  //      outputs [MT][nb][4] bf16 | partials [nb][P][MT][4] | tickets [nb]
  // (48-byte chunk stride: the 12 active lanes of each 16-lane pass of an A read hit 12 distinct 16-byte bank slots of
  // the 256-byte bank row, and the 4 zero-operand lanes read zeros placed in the 4 remaining slots)
  const int tstride = nqs * kCPQ * 96;  // limbs of one token
  uint8_t* xq = lds + 512;
  i32x4* meta = reinterpret_cast<i32x4*>(xq + MT * tstride);
  uint16_t* yl = reinterpret_cast<uint16_t*>(meta + MT * nqs * 4);
  float* part = reinterpret_cast<float*>(yl + ((MT * nb * 4 + 3) & ~3));
  int* tickets = reinterpret_cast<int*>(part + (SPLIT > 1 ? nb * P * MT * 4 : 0));

  if (SPLIT > 1)
    for (int i = tid; i < nb; i += 64 * nwv) tickets[i] = 0;
  if (tid < 128) reinterpret_cast<uint32_t*>(lds)[tid] = 0u;

  // ---- activations, step 1: this lane's bf16 inputs, requested before any weight request (behind the weight requests
  // of the whole GPU, x would arrive microseconds late); the set-up below and the first weight requests overlap x's
  // round trip
  const int gpt = nqs * 4;  // groups per token (of the image)
  const int sub = lane % LPU, units = gpt * MT, ustride = nwv * UPW;
  const int u0 = wave * UPW + lane / LPU;
  const int npass = (units + ustride - 1) >> (lg_nwv + (UPW == 4 ? 2 : 0));
  static_assert(UPW == 4, "four units per wave");
  uint4 xv[XB];
  // ACT: x is gate_up [mm][2k], the activation SiLU(gate) * up of the two halves (the same value as ak_silu_mul's)
  constexpr bool act = ACT;
  const int xk = act ? 2 * k : k;  // x's token stride
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.x), (short)0, mm * xk * 2, kRsrcWord3);
  (void)rx;
  const bool tagged = CHAIN && a.xtg != nullptr;
  const __amdgpu_buffer_rsrc_t rxt =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(a.xtg), (short)0, mm * xk * 4, kRsrcWord3);
  (void)rxt;
  const uint32_t tag2 = (tag & kTagMask) * 0x10001u;
  // the lane's four input pairs of the group at element offset o from the tagged copy: values in v, and whether every
  // word carries the tag.  cached: read through the L2 (the XCD's workgroups share one request to the memory side; a
  // stale line there fails the tag check, and the retries read device-coherently)
  auto ld_tagged = [&](int o, uint4& v, bool cached) __attribute__((always_inline)) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    uint32_t lo[4], hi[4];
    if constexpr (BITS == 4) {
      const int b = (o + unit_pair_offset<4>(sub, 0)) * 4;
      const u32x4 d0 = cached ? __builtin_amdgcn_raw_buffer_load_b128(rxt, b, 0, 0)
                              : __builtin_amdgcn_raw_buffer_load_b128(rxt, b, 0, kSc1);
      const u32x4 d1 = cached ? __builtin_amdgcn_raw_buffer_load_b128(rxt, b + 16, 0, 0)
                              : __builtin_amdgcn_raw_buffer_load_b128(rxt, b + 16, 0, kSc1);
      lo[0] = d0[0], hi[0] = d0[1], lo[1] = d0[2], hi[1] = d0[3];
      lo[2] = d1[0], hi[2] = d1[1], lo[3] = d1[2], hi[3] = d1[3];
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int ob = (o + unit_pair_offset<BITS>(sub, c)) * 4;
        const u32x2 d = cached ? __builtin_amdgcn_raw_buffer_load_b64(rxt, ob, 0, 0)
                               : __builtin_amdgcn_raw_buffer_load_b64(rxt, ob, 0, kSc1);
        lo[c] = d[0], hi[c] = d[1];
      }
    }
    bool ok = true;
    uint32_t w[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      w[c] = __builtin_amdgcn_perm(hi[c], lo[c], 0x05040100u);                   // the two values
      ok = ok && __builtin_amdgcn_perm(hi[c], lo[c], 0x07060302u) == tag2;     // the two tags
    }
    v = make_uint4(w[0], w[1], w[2], w[3]);
    return ok;
  };
  auto xload = [&](int pass0) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      // lanes and passes past the end select zeros.  One launch per step: they load from x[0] (cached; unconditional
      // loads, which the compiler counts exactly, so that it waits for x alone, not for the weights requested after
      // it).  Chained: passes past the end load nothing (x's loads are device-coherent, the last requests of the
      // step; thousands of them at one address would queue at the memory side)
      const int u = u0 + (pass0 + b) * ustride, t = MT == 1 ? 0 : u / gpt, gk = (4 * q0 + u - t * gpt) * kG;
      const bool ok = u < units && t < mm && gk < k;
      xv[b] = make_uint4(0u, 0u, 0u, 0u);
      if (!CHAIN || pass0 + b < npass) {
        const int xo = ok ? t * xk + gk : 0;  // the unit's group
        if constexpr (CHAIN) {  // device-coherent: x may be an earlier step's output, written by another XCD
          auto ld = [&](int o) {
            if constexpr (BITS == 4) {
              const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, (o + unit_pair_offset<4>(sub, 0)) * 2, 0, kSc1);
              return make_uint4(v[0], v[1], v[2], v[3]);
            } else {
              uint32_t v[4];
#pragma unroll
              for (int c = 0; c < 4; ++c)
                v[c] = __builtin_amdgcn_raw_buffer_load_b32(rx, (o + unit_pair_offset<BITS>(sub, c)) * 2, 0, kSc1);
              return make_uint4(v[0], v[1], v[2], v[3]);
            }
          };
          uint4 g = ld(xo);
          if (act) g = silu_mul8(g, ld(xo + k));
          xv[b] = ok ? g : make_uint4(0u, 0u, 0u, 0u);
        } else {
          uint4 g = load_unit<BITS>(a.x + xo, sub);
          if (act) g = silu_mul8(g, load_unit<BITS>(a.x + xo + k, sub));
          xv[b] = ok ? g : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
  };
  // a tagged step's activations of pass pass0 + b, reloaded until all of the wave's words carry the launch's tag (a
  // bounded wait: past it the chain's error flag is raised and the step goes on); one pass at a time, so that only
  // one pass's tagged words are held in registers
  // (pre: the first attempt's words of the first NPRE passes were requested by xpre, before the step's first
  // weights: a step's last workgroup to start is the one the step waits for, and its activations must not return
  // behind its own weight requests; two tokens take two passes at k = 5120)
  constexpr int NPRE = MT == 1 ? 1 : 2;
  uint4 pre_g[NPRE], pre_h[NPRE];
  bool pre_got[NPRE];
  auto xpre = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < NPRE; ++b) {
      const int u = u0 + b * ustride, t = MT == 1 ? 0 : u / gpt, gk = (4 * q0 + u - t * gpt) * kG;
      const bool ok = u < units && t < mm && gk < k;
      pre_g[b] = pre_h[b] = make_uint4(0u, 0u, 0u, 0u);
      pre_got[b] = false;
      if (b < npass && wave * UPW + b * ustride < units) {  // the wave has units in pass b (uniform)
        pre_got[b] = ld_tagged(ok ? t * xk + gk : 0, pre_g[b], AK_TAG_CACHED_FIRST);
        if (act) pre_got[b] = ld_tagged((ok ? t * xk + gk : 0) + k, pre_h[b], AK_TAG_CACHED_FIRST) && pre_got[b];
      }
    }
  };
  auto xpoll = [&](int pass0, int b, bool pre) __attribute__((always_inline)) {
    const int u = u0 + (pass0 + b) * ustride, t = MT == 1 ? 0 : u / gpt, gk = (4 * q0 + u - t * gpt) * kG;
    const bool ok = u < units && t < mm && gk < k;
    xv[b] = make_uint4(0u, 0u, 0u, 0u);
    if (pass0 + b >= npass) return;
    const int xo = ok ? t * xk + gk : 0;
    const long long t0 = wall_clock64();
    bool first = pre;
    for (;;) {
      uint4 g, h2;
      bool got;
      if (first) {
        g = pre_g[b < NPRE ? b : 0], h2 = pre_h[b < NPRE ? b : 0], got = pre_got[b < NPRE ? b : 0];
        first = false;
      } else {
        got = ld_tagged(xo, g, false);
        if (act) got = ld_tagged(xo + k, h2, false) && got;
      }
      if (__all(got || !ok)) {
        if (act) g = silu_mul8(g, h2);
        xv[b] = ok ? g : make_uint4(0u, 0u, 0u, 0u);
        break;
      }
      if (wall_clock64() - t0 > kChainSpinTicks) {
        if ((threadIdx.x & 63) == 0) __hip_atomic_store(&g_chain_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  };
  // the activations of passes pass0 .. pass0 + XB - 1 (pre: passes 0 .. NPRE - 1, requested by xpre)
  auto xload_wait = [&](int pass0, bool pre) __attribute__((always_inline)) {
    if (!tagged) {
      xload(pass0);
      return;
    }
#pragma unroll
    for (int b = 0; b < XB; ++b) xpoll(pass0, b, pre && b < NPRE);
  };
  // a chained step that depends on earlier steps requests its first weights before it waits for them (below)
  const bool late_x = CHAIN && (wait || tagged);
  if (!late_x) xload(0);

  // ---- this wave's tasks: stripe set j, tiles [ta, tb), blocks b0w, b0w + bstep, ... < nb
  constexpr int LGS = SPLIT == 1 ? 0 : SPLIT == 2 ? 1 : SPLIT == 4 ? 2 : 3;
  const int j = wave % SPLIT, bstep = nwv >> LGS, b0w = wave / SPLIT;
  const int pa = SK ? psk : j * P / SPLIT, pb = SK ? psk + 1 : (j + 1) * P / SPLIT;
  const int ta = stripe_tile(pa), tb = stripe_tile(pb);
  const int ntw = b0w < nb ? (nb - b0w + bstep - 1) >> (lg_nwv - LGS) : 0;
  const int nitems = ntw * (tb - ta);
  // stripe ends: a.ends (bit t: tile t ends a stripe; at most 64 tiles without split-K); a split-K wave has one
  // stripe, which ends at tile tb - 1
  const unsigned long long ends = a.ends;

  // ---- weight addressing: per lane fixed, per item scalar.  Rows past the segment's end (padding of the last block)
  // read other rows or, past the buffer, zeros; their results are not written.
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(AK_PICK(sg, sgs.wt)), (short)0, ntile * n * REC, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(AK_PICK(sg, sgs.st)), (short)0, ntile * n * 16, kRsrcWord3);
  // W4: chunk 4 vv + h of each quad; W2 / W3: the chunk pair of group vv + 4 (h & 1) starting at chunk 2 (h >> 1)
  const int cp = 4 * (vv + 4 * (h & 1)) + 2 * (h >> 1);
  const int vo_w = rr * REC + (BITS == 4 ? (4 * vv + h) * 16 : cp * 8), vo_h = rr * REC + 256 + cp * 4;
  const int vo_s = rr * 16 + (vv & 2) * 2;
  const int tile_w = n * REC, tile_s = n * 16;
  auto fetch = [&](int blk, int t, TileRaw<BITS>& d) {
    const int row0 = (b_lo + blk) * 4;
    const int so = row0 * REC + t * tile_w;
    if constexpr (BITS == 4) {
      const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, so, kNt);
      const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, so + 256, kNt);
      d.q0 = make_uint4(v0[0], v0[1], v0[2], v0[3]);
      d.q1 = make_uint4(v1[0], v1[1], v1[2], v1[3]);
    } else {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, so, kNt);
      d.lo = make_uint4(v[0], v[1], v[2], v[3]);
      if constexpr (BITS == 3) {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 g = __builtin_amdgcn_raw_buffer_load_b64(rw, vo_h, so, kNt);
        d.hi = make_uint2(g[0], g[1]);
      }
    }
    // the aligned dwords holding the scales (the item selects the halves): a 16-bit value would be widened or packed
    // at the loop latch, which waits for the load
    const int ss = row0 * 16 + t * tile_s;
    d.s0 = __builtin_amdgcn_raw_buffer_load_b32(rs, vo_s, ss, 0);
    d.s1 = __builtin_amdgcn_raw_buffer_load_b32(rs, vo_s, ss + 8, 0);
  };

  TileRaw<BITS> buf[DEPTH];

  // fetch cursor (an item past the end reloads tile ta of block 0: cache-resident, never used, and the load sequence
  // stays branch-free so the compiler's load counters stay exact)
  int fb = b0w, ft = ta;
  auto fetch_next = [&](TileRaw<BITS>& dst) {
    const bool in = fb < nb;
    fetch(in ? fb : 0, in ? ft : ta, dst);
    const bool wrap = ft + 1 == tb;
    ft = wrap ? ta : ft + 1;
    fb = wrap ? fb + bstep : fb;
  };

  // ---- the first DEPTH items are requested, then step 2 of the activations: per group the limbs (to LDS), and in
  // meta the bias sums -OFF * sum(d_j) of the three limbs with the activation scale 2^(E - 148) as float bits
  if (wait && late_x && wave == 0) chain_poll(target);
  // tagged: AK_TAG_PREFETCH of the DEPTH first items are requested before the activations are waited for, the rest
  // after them
  constexpr int NPF = AK_TAG_PREFETCH < DEPTH ? AK_TAG_PREFETCH : DEPTH;
  if (tagged) xpre();
#pragma unroll
  for (int d = 0; d < DEPTH; ++d)
    if (!tagged || d < NPF) fetch_next(buf[d]);
  if (late_x) {
    if (wait) lds_barrier();
    xload_wait(0, tagged);
  }
  if (tagged) {
#pragma unroll
    for (int d = NPF; d < DEPTH; ++d) fetch_next(buf[d]);
  }

  auto convert = [&](int p0) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      if (p0 + b >= npass || wave * UPW + (p0 + b) * ustride >= units) break;  // no unit of this wave (uniform)
      const int u = u0 + (p0 + b) * ustride;
      const bool live = u < units;
      const int t = MT == 1 || !live ? 0 : u / gpt, ut = live ? u - t * gpt : 0;
      const int qd = ut >> 2, gq = ut & 3, eg0 = 8 * sub, cqd = gq * 4 + (eg0 >> 5);
      int b0, b1, b2;
      const int e = convert_unit<BITS>(xv[b], xq + t * tstride + qd * kCPQ * 96 + cqd * 48, kCPQ * 48, sub & 3, live,
                                       b0, b1, b2);
      if (live) {
        if (sub == 0) {
          constexpr int OFF = code_offset<BITS>();
          const i32x4 mv = {-OFF * b0, -OFF * b1, -OFF * b2, act_scale_bits(e)};
          meta[u] = mv;
        }
      }
    }
  };
  convert(0);
  for (int p0 = XB; p0 < npass; p0 += XB) {
    xload_wait(p0, false);
    convert(p0);
  }
  __syncthreads();

  // A role: group c >> 2, limb c & 3 (limb 3 reads zeros), chunk 4 * (c >> 2) + h of the quad; half 1 is kCPQ * 48
  // bytes further
  const bool a_on = (c & 3) < 3;
  const int a_base = a_on ? 512 + (4 * (c >> 2) + h) * 48 + 16 * (c & 3) : ((c >> 2) * 64 + 48 + h * 48) & 255;
  const int a_qmul = a_on ? kCPQ * 96 : 0, a_tmul = a_on ? tstride : 0;

  // outputs are staged in LDS and written after the loop: a global store among the streaming loads would make the
  // compiler drain every load in flight
  auto write_y = [&](int bl, int t, float y) {  // lanes 0..3: row `lane` of local block bl, token t
    if (lane < 4) yl[(t * nb + bl) * 4 + lane] = f2bf(y);
  };

  // the scale's half of the loaded dword into the high half of an fp32 (v_perm selector per lane), and the source
  // lanes of a stripe partial's four slots (ds_bpermute byte addresses), both loop-invariant
  const uint32_t ssel = vv & 1 ? 0x07060C0Cu : 0x05040C0Cu;
  const int r4 = 4 * (lane & 3);
  const int sl0 = 4 * r4, sl1 = 4 * (17 + r4), sl2 = 4 * (34 + r4), sl3 = 4 * (51 + r4);

  // compute cursor: block, tile, stripe
  int cb = b0w, ct = ta, cs = pa;
  float acc[MT], yrun[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.f, yrun[t] = 0.f;
  // one item without branches: an[] = the accumulators before a stripe end reset them (used only at a stripe end)
  auto core = [&](const TileRaw<BITS>& bf, float (&an)[MT], bool& end, int& eg, int& ep) {
    end = SK ? ct + 1 == tb : ((ends >> ct) & 1ull) != 0;
    Raw<BITS> rq[2];
    split_tile<BITS>(bf, rq[0], rq[1]);
#pragma unroll
    for (int qq = 0; qq < 2; ++qq) {
      i32x4 b0, b1;
      const uint32_t sraw = qq ? bf.s1 : bf.s0;
      const float sc = __uint_as_float(__builtin_amdgcn_perm(sraw, sraw, ssel));
      make_b<BITS>(rq[qq], b0, b1);
      const int cq = 2 * ct + qq;
      // token by token: the activation operand and meta of one token are live at a time
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const i32x4 mt = meta[(t * nqs + cq - q0) * 4 + h];
        const uint8_t* src = lds + a_base + t * a_tmul + (cq - q0) * a_qmul;
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(src);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(src + (a_on ? kCPQ * 48 : 0));
        i32x4 d = mt;
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
        acc[t] = fmaf(group_sum_f32(d), sc * __int_as_float(mt[3]), acc[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      an[t] = acc[t];
      acc[t] = end ? 0.f : acc[t];
    }
    eg = cb;
    ep = cs;
    cs = end ? cs + 1 : cs;
    const bool wrap = ct + 1 == tb;
    ct = wrap ? ta : ct + 1;
    cb = wrap ? cb + bstep : cb;
    cs = wrap ? pa : cs;
  };
  // a stripe ended with accumulators v[]: its partial per row (lanes 0..3: ((slot 0 + slot 1) + slot 2) + slot 3,
  // slot v of row r in lane 17v + 4r), then the blocks' outputs when the task ends
  auto stripe_end = [&](const float (&v)[MT], int eg, int ep) {
    float pp[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int vi = __float_as_int(v[t]);
      const float v0 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl0, vi)),
                  v1 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl1, vi)),
                  v2 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl2, vi)),
                  v3 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl3, vi));
      pp[t] = ((v0 + v1) + v2) + v3;
    }
    if constexpr (SK) {  // to the range's partials, device-coherent (the range's last workgroup adds them)
#pragma unroll
      for (int t = 0; t < MT; ++t)
        if (lane < 4)
          __hip_atomic_store(a.part + ((size_t)(ep * MT + t) * n_b4 + b_lo + eg) * 4 + lane, pp[t], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    } else if constexpr (SPLIT == 1) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        yrun[t] = ep == 0 ? pp[t] : yrun[t] + pp[t];
        if (ep == P - 1) write_y(eg, t, yrun[t]);
      }
    } else {
#pragma unroll
      for (int t = 0; t < MT; ++t)
        if (lane < 4) part[((eg * P + ep) * MT + t) * 4 + lane] = pp[t];
      if (ep + 1 < pb) return;  // more stripes in this task
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  // LDS only: no wait for loads in flight
      int last = 0;
      if (lane == 0) last = atomicAdd(&tickets[eg], 1) == SPLIT - 1;
      last = __shfl(last, 0);
      if (last) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        const float* slot = part + eg * P * MT * 4;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float y = slot[t * 4 + (lane & 3)];
          for (int q = 1; q < P; ++q) y += slot[(q * MT + t) * 4 + (lane & 3)];
          write_y(eg, t, y);
        }
      }
    }
  };

  const int nfull = nitems / DEPTH * DEPTH;
  for (int i0 = 0; i0 < nfull; i0 += DEPTH) {
    float sv[DEPTH][MT];
    bool end[DEPTH];
    int eg[DEPTH], ep[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      core(buf[d], sv[d], end[d], eg[d], ep[d]);
      fetch_next(buf[d]);
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (end[d]) stripe_end(sv[d], eg[d], ep[d]);
  }
  // the last, partial group (its later fetches load the cache-resident dummy item)
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    if (nfull + d < nitems) {
      float v[MT];
      bool e;
      int g, p;
      core(buf[d], v, e, g, p);
      if (e) stripe_end(v, g, p);
    }
  }
  __syncthreads();
  if constexpr (SK) {
    // every wave's partial stores are acknowledged at device scope before the range's counter moves
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    int* const last = reinterpret_cast<int*>(lds);  // the zeros are no longer read
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(a.cnt + r, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last = old == P - 1;
      if (old == P - 1) __hip_atomic_store(a.cnt + r, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
    }
    __syncthreads();
    if (!*last) {
      return;
    }
    for (int i = tid; i < MT * nb * 4; i += 64 * nwv) {
      const int t = MT == 1 ? 0 : i / (nb * 4), o = i - t * nb * 4;
      const size_t off = ((size_t)t * n_b4 + b_lo) * 4 + o;
      yl[i] = f2bf(sum_stripe_partials(a.part, off, (size_t)MT * n_b4 * 4, P));
    }
    __syncthreads();
  }
  for (int i = tid; i < MT * nb * 4; i += 64 * nwv) {
    const int t = MT == 1 ? 0 : i / (nb * 4), row = b_lo * 4 + i - t * nb * 4;
    if (t < mm && row < n) {
      if constexpr (CHAIN) {
        __hip_atomic_store(yseg + (size_t)t * ldy + row, yl[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ytg)
          __hip_atomic_store(ytg + (size_t)t * ldy + row, (uint32_t)yl[i] | ((tag & kTagMask) << 16), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      } else
        yseg[(size_t)t * ldy + row] = yl[i];
    }
  }
}

template <int BITS, int SPLIT, int DEPTH, int MT, bool SK = false, bool ACT = false>
__global__ void __launch_bounds__(1024, 1) i8_m1d_kernel(const I8Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  m1d_body<BITS, SPLIT, DEPTH, MT, false, SK, ACT>(a, lds, false, 0u, 0u);
}

size_t m1d_x_bytes(int nquad, int mt) { return 512 + (size_t)mt * nquad * (kCPQ * 96 + 4 * 16); }
size_t m1d_block_bytes(int P, int split, int mt) {  // per 4-row block: outputs, partials, ticket
  return (size_t)mt * 8 + (split > 1 ? (size_t)P * 16 * mt + 4 : 0);
}

// Launch shape of one GEMV step: workgroups per segment (about the same number of 4-row blocks each, at most one
// workgroup per CU), waves per workgroup and stripe sets per block (SPLIT).  chain: 16 waves (a chained launch has one
// block size).  Returns AK_INVALID if the shape does not suit the kernel.
struct M1dShape {
  int split, nwv, grid;
  size_t smem;
};

// ---- launch configurations pinned by measurement (wq_launch_table.h, written by tune_launch.py) and the tuner's
// override.  A pin names a shape -- bits, padded tokens, k, the segments' rows -- and the stripe sets per block
// (split), waves per workgroup (nwv) and split-K across workgroups (sk) measured fastest for it, and the fastest split
// with 16 waves (csplit: a chained launch always has 16); every configuration gives the same bits, so a pin changes
// only the speed.  Shapes without a pin take the cost model below.
struct M1dPin {
  int bits, mt, k, nseg, n[4];
  int split, nwv, sk, csplit;
};
#include "wq_launch_table.h"

// The tuner's process-global override (ak_wq_tune_override): atomics, so that a launch on another thread reads each
// field whole (tuning only: a launch during a change may see some fields before it and some after it)
struct TuneOverride {
  std::atomic<int> split{0}, nwv{0}, sk{-1};  // 0 / -1: not overridden
  std::atomic<bool> nopins{false};            // the cost model alone (the tuner's reference)
};
TuneOverride g_tune;

const M1dPin* find_pin(const I8Args& a, int bits, int mt) {
  if (g_tune.nopins) return nullptr;
  const Segs& g = a.segs;
  for (int i = 0; i < (int)(sizeof(kM1dPins) / sizeof(kM1dPins[0])); ++i) {
    const M1dPin& p = kM1dPins[i];
    if (p.bits != bits || p.mt != mt || p.k != a.k || p.nseg != g.nseg) continue;
    bool same = true;
    for (int j = 0; j < g.nseg; ++j) same = same && p.n[j] == g.n[j];
    if (same) return &p;
  }
  return nullptr;
}

// split-K across workgroups: -1 the default rule (wherever the shape suits it), 0 no, 1 yes
int m1d_sk_choice(const I8Args& a, int bits, int mt) {
  if (g_tune.sk >= 0) return g_tune.sk;
  const M1dPin* p = find_pin(a, bits, mt);
  return p && p->sk >= 0 ? p->sk : -1;
}

int plan_m1d(I8Args& a, int bits, int mt, bool chain, M1dShape& sh) {
  const Segs& g = a.segs;
  const size_t x_bytes = m1d_x_bytes(a.nquad, mt);
  const int ntile = a.nquad / 2;
  for (int i = 0; i < g.nseg; ++i)  // buffer offsets are 32-bit
    if ((long long)ntile * g.n[i] * 128 * bits >= (1ll << 31)) return AK_INVALID;
  if (x_bytes > 150 * 1024 || a.nquad / 2 > 64) return AK_INVALID;  // (the stripe-end mask covers 64 tiles)
  int total = 0;
  for (int i = 0; i < g.nseg; ++i) total += (g.n[i] + 3) / 4;
  const int cus = num_cus();
  int per = (total + cus - 1) / cus, grid = 0;
  for (;; ++per) {
    grid = 0;
    for (int i = 0; i < g.nseg; ++i) grid += ((g.n[i] + 3) / 4 + per - 1) / per;
    if (grid <= cus || per >= total) break;
  }
  for (int i = 0, e = 0; i < kMaxSegs; ++i) {
    if (i < g.nseg) e += ((g.n[i] + 3) / 4 + per - 1) / per;
    a.wg_end[i] = e;
  }
  int nbmax = 0;
  for (int i = 0; i < g.nseg; ++i) {
    const int nbs = (g.n[i] + 3) / 4, gs = (nbs + per - 1) / per;
    nbmax = (nbs + gs - 1) / gs > nbmax ? (nbs + gs - 1) / gs : nbmax;
  }
  // waves per workgroup and waves per block: fewest item rounds for the busiest wave, a task's overhead counted as
  // about half an item; ties go to more waves (latency hiding) and fewer waves per block (less exchange)
  int best_split = 1, best_nwv = 16;
  double best = 1e30;
  for (int nwv : {16, 8}) {
    if (chain && nwv != 16) continue;
    for (int split : {1, 2, 4, 8}) {
      if (split > a.P) break;
      if (x_bytes + (size_t)nbmax * m1d_block_bytes(a.P, split, mt) + 16 > 160 * 1024) continue;
      int lmax = 0;
      for (int j = 0; j < split; ++j) {
        const int l = (stripe_begin((j + 1) * a.P / split, a.nquad, a.P, 2) -
                       stripe_begin(j * a.P / split, a.nquad, a.P, 2)) / 2;
        lmax = l > lmax ? l : lmax;
      }
      const int bstep = nwv / split;
      const double cost = (double)((nbmax + bstep - 1) / bstep) * (lmax + 0.5);
      if (cost < best - 1e-9) best = cost, best_split = split, best_nwv = nwv;
    }
  }
  if (best > 1e29) return AK_INVALID;
  // chained steps with at least 8 blocks per workgroup: whole blocks per wave (measured in the chained sweeps: M = 1
  // 2937 -> 2918 us, M = 2 3840 -> 3782 us, one TP = 2 rank 2137 -> 2131 us; from 5 blocks on, TP = 2 got slower)
  constexpr int kChainSplit1Blocks = 8;
  if (chain && nbmax >= kChainSplit1Blocks) best_split = 1;
  // a measured pin (or the tuner's override) replaces the model's choice where the shape admits it
  const M1dPin* pin = find_pin(a, bits, mt);
  // (csplit 0: a chained launch keeps the model's split)
  const int o_split = g_tune.split.load(std::memory_order_relaxed), o_nwv = g_tune.nwv.load(std::memory_order_relaxed);
  const int want_split = o_split ? o_split : pin ? (chain ? pin->csplit : pin->split) : 0;
  const int want_nwv = o_nwv ? o_nwv : pin ? pin->nwv : 0;
  if (want_split || want_nwv) {
    const int sp = want_split ? want_split : best_split, nw = chain ? 16 : want_nwv ? want_nwv : best_nwv;
    const bool ok = (sp == 1 || sp == 2 || sp == 4 || sp == 8) && sp <= a.P && (nw == 16 || nw == 8) &&
                    x_bytes + (size_t)nbmax * m1d_block_bytes(a.P, sp, mt) + 16 <= 160 * 1024;
    if (ok) best_split = sp, best_nwv = nw;
  }
  sh.split = best_split;
  sh.nwv = best_nwv;
  sh.grid = grid;
  sh.smem = x_bytes + (size_t)nbmax * m1d_block_bytes(a.P, best_split, mt) + 16;
  return 0;
}

constexpr int m1d_depth(int mt) { return mt <= 2 ? AK_M1_TILES : 1; }  // items in flight per wave

template <int BITS, int SPLIT, int MT, bool ACT>
void launch_split(const I8Args& a, int grid, int nwv, size_t smem, hipStream_t s) {
  hipLaunchKernelGGL((i8_m1d_kernel<BITS, SPLIT, m1d_depth(MT), MT, false, ACT>), dim3(grid), dim3(64 * nwv), smem, s,
                     a);
}

// split-K across workgroups (one segment, 8 stripes, k of at least AK_M1_SK_QUADS quads): P workgroups per row range,
// each one stripe; partials and counters in the stream's scratch.  0: not launched (no scratch inside a capture, or
// the shape does not suit it).
#ifndef AK_M1_SK_QUADS
#define AK_M1_SK_QUADS 32
#endif
// the split-K shape of a launch: row ranges nr, LDS bytes and scratch bytes (4 KB of counters, then the partials);
// false if the launch does not suit it
bool m1d_sk_shape(const I8Args& a, int bits, int mt, int* nr_out, size_t* smem_out, size_t* scratch_out) {
  const Segs& g = a.segs;
  const int choice = m1d_sk_choice(a, bits, mt);
  if (choice == 0) return false;
  if (mt > 2 || g.nseg != 1 || a.P != 8 || (a.nquad < AK_M1_SK_QUADS && choice != 1)) return false;
  if ((long long)(a.nquad / 2) * g.n[0] * 128 * bits >= (1ll << 31)) return false;
  const int cus = num_cus(), nr = cus / a.P, nb4 = (g.n[0] + 3) / 4, nbr = nr > 0 ? (nb4 + nr - 1) / nr : 0;
  int nqs = 0;
  for (int p = 0; p < a.P; ++p) {
    const int q = stripe_begin(p + 1, a.nquad, a.P, 2) - stripe_begin(p, a.nquad, a.P, 2);
    nqs = q > nqs ? q : nqs;
  }
  const size_t smem = m1d_x_bytes(nqs, mt) + (size_t)nbr * m1d_block_bytes(a.P, 1, mt) + 16;
  if (nr < 1 || nr > 1024 || smem > 160 * 1024) return false;
  *nr_out = nr;
  *smem_out = smem;
  *scratch_out = 4096 + (size_t)a.P * mt * nb4 * 4 * 4;
  return true;
}

template <int BITS, int MT, bool ACT>
int launch_m1d_sk(I8Args a, hipStream_t s) {
  if constexpr (MT > 2) return AK_INVALID;  // 3..8 tokens: the tokens-in-A-rows kernel has its own split
  int nr = 0;
  size_t smem = 0, zb = 0;
  if (!m1d_sk_shape(a, BITS, MT, &nr, &smem, &zb)) return AK_INVALID;
  void* z = stream_scratch(s, zb);
  if (!z) return AK_INVALID;
  a.cnt = static_cast<int*>(z);
  a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(z) + 4096);
  a.wg_end[0] = nr * a.P;
  hipLaunchKernelGGL((i8_m1d_kernel<BITS, 1, m1d_depth(MT), MT, true, ACT>), dim3(nr * a.P), dim3(1024), smem, s, a);
  return (int)hipGetLastError();
}

template <int BITS, int MT, bool ACT>
int launch_m1d_act(I8Args a, hipStream_t s) {
  if (launch_m1d_sk<BITS, MT, ACT>(a, s) != AK_INVALID) return (int)hipGetLastError();
  M1dShape sh;
  if (plan_m1d(a, BITS, MT, false, sh)) return AK_INVALID;
  switch (sh.split) {
    case 1: launch_split<BITS, 1, MT, ACT>(a, sh.grid, sh.nwv, sh.smem, s); break;
    case 2: launch_split<BITS, 2, MT, ACT>(a, sh.grid, sh.nwv, sh.smem, s); break;
    case 4: launch_split<BITS, 4, MT, ACT>(a, sh.grid, sh.nwv, sh.smem, s); break;
    default: launch_split<BITS, 8, MT, ACT>(a, sh.grid, sh.nwv, sh.smem, s); break;
  }
  return (int)hipGetLastError();
}

template <int BITS, int MT>
int launch_m1d(I8Args a, hipStream_t s) {
  return a.act ? launch_m1d_act<BITS, MT, true>(a, s) : launch_m1d_act<BITS, MT, false>(a, s);
}

// ---- chained launches: one persistent workgroup per CU runs the steps in order
constexpr int kSplitK = 256, kAct = 512, kChainLean = 16;
struct ChainStep {
  I8Args a;
  int kind;  // bits * 16 + SPLIT, + kSplitK for a split-K step, + kAct for a split-K step with SiLU(gate) * up
  int wait;    // 1: the step reads (or overwrites) what earlier steps wrote or read: wait for all of them
  int signal;  // 1: a later step waits at the grid barrier for this one: signal the flags after it
};

// epochs: one word per workgroup in the chain's memory, the number of launches of this chain so far (every workgroup
// counts every launch, so they agree); the tag of a launch is the low 16 bits of its epoch + 1, which differ from the
// tags the previous launch left in the tagged copies and from their initial zeros
// LEAN: only the step kinds of one- or two-stripe-set steps and plain split-K steps (the decode sweep's): a smaller
// kernel (the chained kernel is sensitive to its code size: the M = 1 sweep 2921-2925 -> 2913-2918 us on one box)
template <int MT, bool LEAN>
__global__ void __launch_bounds__(1024, 1) i8_chain_kernel(const ChainStep* __restrict__ steps, int nsteps,
                                                           uint32_t* __restrict__ epochs) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int D = m1d_depth(MT);
  uint32_t* const flag = g_chain_flags + blockIdx.x * kChainFlagStride;
  // every workgroup's flag holds the same count between chained launches (all of them signal the last step)
  const uint32_t f0 = __builtin_amdgcn_readfirstlane(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const uint32_t ep = __builtin_amdgcn_readfirstlane(epochs[blockIdx.x]);
  const uint32_t tag = (ep + 1u) & kTagMask;
  for (int s = 0; s < nsteps; ++s) {
    const ChainStep st = steps[s];  // a copy: the step's fields live in scalar registers
    const bool w = st.wait != 0;
    const uint32_t target = f0 + (uint32_t)s;
    if constexpr (LEAN) {
      switch (st.kind) {
        case 4 * 16 + 1: m1d_body<4, 1, D, MT, true>(st.a, lds, w, target, tag); break;
        case 4 * 16 + 2: m1d_body<4, 2, D, MT, true>(st.a, lds, w, target, tag); break;
        case 3 * 16 + 1: m1d_body<3, 1, D, MT, true>(st.a, lds, w, target, tag); break;
        case 3 * 16 + 2: m1d_body<3, 2, D, MT, true>(st.a, lds, w, target, tag); break;
        case 2 * 16 + 2: m1d_body<2, 2, D, MT, true>(st.a, lds, w, target, tag); break;
        case kSplitK + 4 * 16 + 1: m1d_body<4, 1, D, MT, true, true>(st.a, lds, w, target, tag); break;
        case kSplitK + 3 * 16 + 1: m1d_body<3, 1, D, MT, true, true>(st.a, lds, w, target, tag); break;
        case kSplitK + 2 * 16 + 1: m1d_body<2, 1, D, MT, true, true>(st.a, lds, w, target, tag); break;
        default: m1d_body<2, 1, D, MT, true>(st.a, lds, w, target, tag); break;
      }
    } else {
      switch (st.kind) {
        case 4 * 16 + 1: m1d_body<4, 1, D, MT, true>(st.a, lds, w, target, tag); break;
        case 4 * 16 + 2: m1d_body<4, 2, D, MT, true>(st.a, lds, w, target, tag); break;
        case 4 * 16 + 4: m1d_body<4, 4, D, MT, true>(st.a, lds, w, target, tag); break;
        case 4 * 16 + 8: m1d_body<4, 8, D, MT, true>(st.a, lds, w, target, tag); break;
        case 3 * 16 + 1: m1d_body<3, 1, D, MT, true>(st.a, lds, w, target, tag); break;
        case 3 * 16 + 2: m1d_body<3, 2, D, MT, true>(st.a, lds, w, target, tag); break;
        case 3 * 16 + 4: m1d_body<3, 4, D, MT, true>(st.a, lds, w, target, tag); break;
        case 3 * 16 + 8: m1d_body<3, 8, D, MT, true>(st.a, lds, w, target, tag); break;
        case 2 * 16 + 1: m1d_body<2, 1, D, MT, true>(st.a, lds, w, target, tag); break;
        case 2 * 16 + 2: m1d_body<2, 2, D, MT, true>(st.a, lds, w, target, tag); break;
        case 2 * 16 + 4: m1d_body<2, 4, D, MT, true>(st.a, lds, w, target, tag); break;
        case kSplitK + 4 * 16 + 1: m1d_body<4, 1, D, MT, true, true>(st.a, lds, w, target, tag); break;
        case kSplitK + 3 * 16 + 1: m1d_body<3, 1, D, MT, true, true>(st.a, lds, w, target, tag); break;
        case kSplitK + 2 * 16 + 1: m1d_body<2, 1, D, MT, true, true>(st.a, lds, w, target, tag); break;
        case kAct + kSplitK + 4 * 16 + 1: m1d_body<4, 1, D, MT, true, true, true>(st.a, lds, w, target, tag); break;
        case kAct + kSplitK + 3 * 16 + 1: m1d_body<3, 1, D, MT, true, true, true>(st.a, lds, w, target, tag); break;
        case kAct + kSplitK + 2 * 16 + 1: m1d_body<2, 1, D, MT, true, true, true>(st.a, lds, w, target, tag); break;
        default: m1d_body<2, 8, D, MT, true>(st.a, lds, w, target, tag); break;
      }
    }
    // signal: this workgroup's outputs of steps <= s are stored (each wave waits for its own stores' acknowledgement,
    // which for sc1 stores means written through to device scope).  Without a signal the workgroup goes on at once
    // (its stores complete in the background; the next step's LDS is reused only after the barrier).
    if (st.signal || s + 1 == nsteps) {
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      __syncthreads();
      if (threadIdx.x == 0) __hip_atomic_store(flag, f0 + (uint32_t)s + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      lds_barrier();
    }
  }
  if (threadIdx.x == 0) epochs[blockIdx.x] = ep + 1u;
}

}  // namespace

// up to 8 tokens (padded to 1, 2, 4 or 8 in the kernel); each segment's rows are processed in 4-row blocks (the last
// one padded).  Returns AK_INVALID if the shape does not suit the kernel (group 64, the tokens' activations beyond the
// LDS, a segment beyond 2 GB): the caller falls back to the any-m kernel.  act = 1: x is the merged gate_up [m][2k] and
// the activations are SiLU(gate) * up.
int i8_gemv_m1(int bits, const void* x, int m, const Segs& g, int k, int group, hipStream_t s, int act) {
  if (group != kG || m < 1 || m > 8) return AK_INVALID;
  I8Args a;
  a.act = act;
  a.segs = g;
  a.x = static_cast<const uint16_t*>(x);
  a.m = m;
  a.k = k;
  a.nquad = kpad(k) / kG / 4;
  a.qpt = 2;
  set_tile_stripes(a);
  a.nb = 0;
  a.part = nullptr;
  a.cnt = nullptr;
  const int mt = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
  switch (bits * 10 + mt) {
    case 41: return launch_m1d<4, 1>(a, s);
    case 31: return launch_m1d<3, 1>(a, s);
    case 21: return launch_m1d<2, 1>(a, s);
    case 42: return launch_m1d<4, 2>(a, s);
    case 32: return launch_m1d<3, 2>(a, s);
    case 22: return launch_m1d<2, 2>(a, s);
    case 44: return launch_m1d<4, 4>(a, s);
    case 34: return launch_m1d<3, 4>(a, s);
    case 24: return launch_m1d<2, 4>(a, s);
    case 48: return launch_m1d<4, 8>(a, s);
    case 38: return launch_m1d<3, 8>(a, s);
    case 28: return launch_m1d<2, 8>(a, s);
    default: return AK_INVALID;
  }
}

// ---- chained launches (host side)

// Table of a chain's steps in device memory, or AK_INVALID if some step does not suit the chained kernel (group 64,
// more than two tokens, activations beyond the LDS, a segment beyond 2 GB): the caller then runs the steps one launch
// each.  x[i], m[i], k[i], bits[i], segs[i], wait[i] describe step i.
int m1d_chain_make(int nsteps, const int* bits, const void* const* x, const int* m, const int* k, const Segs* segs,
                   const int* wait, const int* act, void** table, int* mt_out, size_t* smem_out) {
  int mt = 1;
  for (int i = 0; i < nsteps; ++i) {
    if (m[i] < 1 || m[i] > 2 || bits[i] < 2 || bits[i] > 4) return AK_INVALID;
    mt = m[i] > mt ? m[i] : mt;
  }
  if (num_cus() > kChainMaxWg) return AK_INVALID;
  ChainStep* h = static_cast<ChainStep*>(calloc((size_t)nsteps, sizeof(ChainStep)));
  if (!h) return AK_OOM;
  size_t smem = 0;
  // the table, then (zeroed) the workgroups' epochs, the tagged output copies and the split-K steps' scratch (counters
  // and partials)
  const size_t table_bytes = ((size_t)nsteps * sizeof(ChainStep) + 255) & ~(size_t)255;
  size_t total = table_bytes + kChainMaxWg * 4;
  std::vector<size_t> zoff((size_t)nsteps, 0);
  // tagged waits: step i reads its activations from a tagged copy of segment tseg[i] of step i - 1's outputs where
  // that segment holds all of them (x is its start, its rows dense, m * k of x within its m * n outputs), step i - 1
  // waited for the step before it (or is the first) and step i + 1 waits (or there is none); AK_CHAIN_TAGS=0: never
  std::vector<int> tseg((size_t)nsteps, -1);
  std::vector<size_t> toff((size_t)nsteps, 0);
  const char* ev = getenv("AK_CHAIN_TAGS");
  const bool tags_on = !(ev && atoi(ev) == 0);
  for (int i = 1; i < nsteps && tags_on; ++i) {
    if (!wait[i] || (i > 1 && !wait[i - 1]) || (i + 1 < nsteps && !wait[i + 1])) continue;
    const Segs& p = segs[i - 1];
    const long long need = (long long)m[i] * k[i] * (act[i] ? 2 : 1);
    for (int j = 0; j < p.nseg; ++j)
      if (p.y[j] == x[i] && p.ldy[j] == p.n[j] && need <= (long long)m[i - 1] * p.n[j]) {
        tseg[(size_t)i] = j;
        toff[(size_t)i] = total;
        total += ((size_t)m[i - 1] * p.n[j] * 4 + 255) & ~(size_t)255;
        break;
      }
  }
  for (int i = 0; i < nsteps; ++i) {
    I8Args& a = h[i].a;
    a.segs = segs[i];
    a.x = static_cast<const uint16_t*>(x[i]);
    a.m = m[i];
    a.k = k[i];
    a.nquad = kpad(k[i]) / kG / 4;
    a.qpt = 2;
    set_tile_stripes(a);
    a.nb = 0;
    a.part = nullptr;
    a.cnt = nullptr;
    h[i].wait = i > 0 && wait[i] && tseg[(size_t)i] < 0 ? 1 : 0;
    h[i].signal = i + 1 < nsteps && wait[i + 1] && tseg[(size_t)i + 1] < 0 ? 1 : 0;
    a.act = act[i];
    int nr = 0;
    size_t sks = 0, zb = 0;
    if (m1d_sk_shape(a, bits[i], mt, &nr, &sks, &zb) && nr * a.P <= num_cus()) {
      h[i].kind = (act[i] ? kAct : 0) + kSplitK + bits[i] * 16 + 1;
      a.wg_end[0] = nr * a.P;
      zoff[(size_t)i] = total;
      total += (zb + 255) & ~(size_t)255;
      smem = sks > smem ? sks : smem;
      continue;
    }
    M1dShape sh;
    if (act[i] || plan_m1d(a, bits[i], mt, true, sh)) {  // SiLU(gate) * up steps: split-K shapes only
      free(h);
      return AK_INVALID;
    }
    h[i].kind = bits[i] * 16 + sh.split;
    smem = sh.smem > smem ? sh.smem : smem;
  }
  void* d = nullptr;
  int e = (int)hipMalloc(&d, total);
  if (!e && total > table_bytes) e = (int)hipMemset(static_cast<uint8_t*>(d) + table_bytes, 0, total - table_bytes);
  for (int i = 0; i < nsteps && !e; ++i) {
    if (tseg[(size_t)i] >= 0) {
      uint32_t* tb = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(d) + toff[(size_t)i]);
      h[i].a.xtg = tb;
      h[i - 1].a.ytg[tseg[(size_t)i]] = tb;
    }
    if (zoff[(size_t)i]) {
      h[i].a.cnt = reinterpret_cast<int*>(static_cast<uint8_t*>(d) + zoff[(size_t)i]);
      h[i].a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(d) + zoff[(size_t)i] + 4096);
    }
  }
  bool lean = true;  // every step a kind of the lean kernel
  for (int i = 0; i < nsteps; ++i) {
    const int kd = h[i].kind, sp = kd & 15;
    lean = lean && (kd < kSplitK ? sp == 1 || sp == 2 : kd < kAct && sp == 1);
  }
  if (!e) e = (int)hipMemcpy(d, h, (size_t)nsteps * sizeof(ChainStep), hipMemcpyHostToDevice);
  free(h);
  if (e) {
    if (d) (void)hipFree(d);
    return e == (int)hipErrorOutOfMemory ? AK_OOM : e;
  }
  *table = d;
  *mt_out = mt + (lean ? kChainLean : 0);
  *smem_out = smem;
  return 0;
}

int m1d_chain_launch(const void* table, int nsteps, int mt, size_t smem, hipStream_t s) {
  const ChainStep* t = static_cast<const ChainStep*>(table);
  uint32_t* ep = reinterpret_cast<uint32_t*>(const_cast<uint8_t*>(static_cast<const uint8_t*>(table)) +
                                             (((size_t)nsteps * sizeof(ChainStep) + 255) & ~(size_t)255));
  switch (mt) {  // + kChainLean: every step has a kind of the lean kernel
    case 1: hipLaunchKernelGGL((i8_chain_kernel<1, false>), dim3(num_cus()), dim3(1024), smem, s, t, nsteps, ep); break;
    case 2: hipLaunchKernelGGL((i8_chain_kernel<2, false>), dim3(num_cus()), dim3(1024), smem, s, t, nsteps, ep); break;
    case 1 + kChainLean:
      hipLaunchKernelGGL((i8_chain_kernel<1, true>), dim3(num_cus()), dim3(1024), smem, s, t, nsteps, ep);
      break;
    default:
      hipLaunchKernelGGL((i8_chain_kernel<2, true>), dim3(num_cus()), dim3(1024), smem, s, t, nsteps, ep);
      break;
  }
  return (int)hipGetLastError();
}

// the tuner's override of the launch configuration (0 / -1: the pins and the model)
void m1d_tune_override(int split, int nwv, int sk) {
  g_tune.nopins = sk == -2;
  g_tune.split = split;
  g_tune.nwv = nwv;
  g_tune.sk = sk < -1 ? -1 : sk;
}

// the configuration a one- or two-token launch of this shape takes: split, nwv, sk (1 split-K across workgroups)
int m1d_tune_query(int bits, int m, const Segs& g, int k, int* split, int* nwv, int* sk) {
  if (m < 1 || m > 2 || bits < 2 || bits > 4) return AK_INVALID;
  I8Args a;
  a.segs = g;
  a.x = nullptr;
  a.m = m;
  a.k = k;
  a.nquad = kpad(k) / kG / 4;
  a.qpt = 2;
  set_tile_stripes(a);
  a.nb = 0;
  a.part = nullptr;
  a.cnt = nullptr;
  int nr = 0;
  size_t smem = 0, zb = 0;
  if (m1d_sk_shape(a, bits, m, &nr, &smem, &zb)) {
    *split = 1, *nwv = 16, *sk = 1;
    return 0;
  }
  M1dShape sh;
  if (plan_m1d(a, bits, m, false, sh)) return AK_INVALID;
  *split = sh.split, *nwv = sh.nwv, *sk = 0;
  return 0;
}

// reads and clears the flag a chained launch raises when a wait ran out (0.2 s): 1 if one did since the last call
int m1d_chain_error(int* err) {
  uint32_t v = 0, z = 0;
  int e = (int)hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_chain_err), sizeof(v), 0, hipMemcpyDeviceToHost);
  if (!e && v) e = (int)hipMemcpyToSymbol(HIP_SYMBOL(g_chain_err), &z, sizeof(z), 0, hipMemcpyHostToDevice);
  *err = (int)v;
  return e;
}

}  // namespace agq
