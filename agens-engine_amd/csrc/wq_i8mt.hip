// The default-numerics GEMV for 3..8 tokens (speculative verify, small batches), group 128, on gfx950: the same exact
// integer group sums and the same fp32 combine order as wq_i8.hip / wq_i8m1d.hip (every output row is bit-identical
// to its one-token launch), with the tokens in the rows of the MFMA A operand: one v_mfma_i32_16x16x64_i8 serves
// 4 tokens x 16 output rows instead of 1 token x 4 rows.
//
// MFMA layout (16-row blocks, one group of 128 inputs per pair of MFMAs):
//   lane (c, h) = (lane % 16, lane / 16);
//   B column c = output row c of the block: lane (c, h) holds chunk h of the group (32 inputs; the MFMA pair takes
//     its two 16-input halves);
//   A row c = (token 4 tg + (c >> 2), limb c & 3): lane (c, h) holds that limb of the inputs of chunk h (limb 3 is
//     zero);
//   D: lane (c, h) holds row c x token 4 tg + h, its three limb sums in D[0..2] and, through the C operand (meta), the
//     bias -OFF * sum(d_j) and the token's activation scale in D[3] -- everything a lane needs stays in the lane.
//
// Loads: an item is 16 rows x one quad (512 inputs), loaded in whole lines (8 rows x 128 B per instruction: the two
// lanes of a column pair load the two halves of one row's line, and one DPP swap per dword pair gives each lane its own
// row, quad_pair_rows).  Then W4: one 16-byte chunk per group.  W2 and the W3 two-bit planes: one
// 16-byte chunk pair per lane covers two groups (chunks 2 (h >> 1), 2 (h >> 1) + 1 of group 2 j + (h & 1)); one
// v_permlane16_swap per dword pair (odd 16-lane rows of the first operand <-> even rows of the second) turns it into
// the operands of groups 2 j and 2 j + 1.  The W3 third-bit plane the same with 8-byte pairs.
//
// Activations: converted once per workgroup into LDS in the A-operand order (per group, half, token group and chunk:
// the 12 limb rows of 4 tokens, 16 bytes each, 192 bytes; the 12 active lanes of each 16-lane pass hit 12 distinct
// 16-byte bank slots and the 4 zero-limb lanes read zeros placed at the 4 remaining slots).
//
// Work decomposition as the one-token kernel: one persistent workgroup per CU owns a contiguous range of 16-row
// blocks of one segment; tasks are (block, stripe set), SPLIT per block from a launch-time cost model; a wave keeps
// the accumulators of its task per (token, group slot), adds a stripe's four slots in order in the lane, and partials
// of split blocks meet in LDS where the last task adds them in stripe order.
#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_i8_common.h"
#include "wq_quad.h"

#include <stdlib.h>

#include <vector>

namespace agq {

int num_cus();
void* stream_scratch(hipStream_t s, size_t bytes);

namespace {

constexpr int kG = 128;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, dword 3 (CDNA)
constexpr int kNt = 2;                    // streaming (non-temporal) cache policy for the weights
constexpr int kVmcnt0 = 0x0F70;            // s_waitcnt immediate: vector memory counter 0, the others unconstrained
constexpr int kSc1 = 16;                  // device-scope coherent access (sc1): misses / writes through the L2

// Chained launches of this kernel's steps (3..4 tokens): one persistent workgroup per CU runs the steps in order.  A
// step that reads earlier steps' outputs either waits at a grid barrier (every workgroup's flag word reaches the
// step) or, where its activations are the output of the step just before it, polls a tagged copy of that output
// (32-bit words bf16 | tag << 16, the tag the low 16 bits of the launch count + 1) until every word it reads carries
// the launch's tag.  Outputs are written with device-coherent stores; the steps' own LDS is reused after an LDS-only
// barrier.  Waits are bounded (0.2 s of the wall clock; then the error flag is raised and the step goes on).
constexpr int kMtChainMaxWg = 1024;
constexpr long long kMtChainSpinTicks = 20000000;  // 0.2 s of the 100 MHz wall clock
constexpr uint32_t kMtTagMask = 0xFFFFu;
__device__ __attribute__((aligned(256))) uint32_t g_mt_chain_flags[kMtChainMaxWg];
__device__ uint32_t g_mt_chain_err;

// wave 0 polls until the flags of workgroups [0, nwg) are all at least `target` (wrap-safe), 16 bytes per lane
__device__ __forceinline__ void mt_chain_poll(uint32_t target) {
  const int lane = threadIdx.x, nwg = gridDim.x;
  const long long t0 = wall_clock64();
  const __amdgpu_buffer_rsrc_t rf =
      __builtin_amdgcn_make_buffer_rsrc(g_mt_chain_flags, (short)0, kMtChainMaxWg * 4, kRsrcWord3);
  for (;;) {
    bool ok = true;
    for (int j = 4 * lane; j < nwg; j += 256) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rf, j * 4, 0, kSc1);
#pragma unroll
      for (int i = 0; i < 4; ++i) ok = ok && (j + i >= nwg || (int)(v[i] - target) >= 0);
    }
    if (__all(ok)) break;
    if (wall_clock64() - t0 > kMtChainSpinTicks) {
      if (lane == 0) __hip_atomic_store(&g_mt_chain_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// the workgroup meets at an LDS-only barrier (loads in flight stay in flight)
__device__ __forceinline__ void mt_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// LDS bytes of the activation image (per group: 2 halves x NT token groups x 4 chunks x 192 B) and its meta
__host__ __device__ inline int mt_a_bytes(int ngroups, int nt) { return ngroups * 2 * nt * 768; }
__host__ __device__ inline int mt_meta_bytes(int ngroups, int nt) { return nt * ngroups * 4 * 16; }

// CH: the stripes are processed in a.nb chunks one after the other (all waves on one chunk's stripes, each chunk with
// its own activation image), for activations beyond the LDS; stripe partials wait in the LDS and are added in stripe
// order at the end, so the results are those of an unchunked launch.
//
// SK (split-K across workgroups, for activations beyond the LDS, one segment): workgroup (r, p) computes stripe p of the
// rows of range r, converting only that stripe's activations; it writes its stripe partials with device-coherent
// stores, and the last of the range's P workgroups (device-scope counter) adds them in stripe order and writes y.
// ACT (split-K launches only): x is the merged gate_up [m][2k], the activations SiLU(gate) * up (ak_silu_mul's value)
//
// TH (split-K only, one segment, 9..16 tokens as NT = 2): the launch holds two token halves, workgroups [0, W) for
// tokens 0..7 and [W, 2W) for tokens 8.. (W = a.wg_end[3]); each half computes exactly what the 8-token launch of its
// tokens computes, with its own stripe partials and counters.
// CHAIN (whole-image and split-K steps, no SiLU(gate) * up): a step of a chained launch (see mt_chain_poll): workgroups
// past the step's grid return at once (after the step's wait); the activations are requested after the step's first
// weights and its wait, device-coherently or from the tagged copy a.xtg; outputs are stored device-coherently, with
// their tagged copy where a.ytg asks for it.
template <int BITS, int SPLIT, int DEPTH, int NT, bool CH, bool SK = false, bool ACT = false, bool TH = false,
          bool CHAIN = false>
__device__ __forceinline__ void mt_body(const I8Args& a, uint8_t* lds, bool wait, uint32_t target, uint32_t tag) {
  static_assert(!TH || (SK && NT == 2), "token halves: split-K launches of 8-token halves");
  static_assert((!CH && !SK) || SPLIT == 1, "chunked and split launches give every wave whole stripes of its blocks");
  static_assert(!(CH && SK), "one of the two");
  static_assert(!CHAIN || (!CH && !TH && !ACT), "chained steps: whole-image or split-K launches");
  constexpr int LPU = kG / 8, UPW = 64 / LPU, XB = 4, MP = 4 * NT;  // MP: padded tokens
  constexpr int REC = 128 * BITS;
  const int P = a.P, nquad = a.nquad, k = a.k;
  const int thw = TH ? a.wg_end[kMaxSegs - 1] : 0, th = TH && (int)blockIdx.x >= thw ? 1 : 0;
  const int bid = (int)blockIdx.x - th * thw;  // the workgroup's index within its token half
  const int mm = TH ? (th ? a.m - 8 : 8) : a.m;
  const uint16_t* const xb = a.x + (TH ? (size_t)th * 8 * (ACT ? 2 * k : k) : 0);
  const int ngroups = nquad * 4;
  const int nwv = blockDim.x >> 6;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Segs& sgs = a.segs;
  if constexpr (CHAIN) {
    if ((int)blockIdx.x >= AK_PICK(sgs.nseg - 1, a.wg_end)) {  // no rows in this step
      if (wait && wave == 0) mt_chain_poll(target);
      return;
    }
  }

  // this workgroup's segment and its 16-row blocks [b_lo, b_lo + nb) of that segment (SK: row range r, stripe psk)
  int sg = 0;
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) sg += (i < sgs.nseg && bid >= a.wg_end[i - 1]) ? 1 : 0;
  // (SK: segment i has (wg_end[i] - wg_end[i-1]) / P row ranges; range r of the segment is counter wg0 / P + r, its
  // partials start after the earlier segments')
  const int wg0 = sg ? AK_PICK(sg - 1, a.wg_end) : 0, li = bid - wg0;
  const int nr = SK ? (AK_PICK(sg, a.wg_end) - wg0) / P : 1, r = SK ? li / P : 0, psk = SK ? li - r * P : 0;
  const int gs = SK ? nr : AK_PICK(sg, a.wg_end) - wg0, w = SK ? r : li;
  const int n = AK_PICK(sg, sgs.n), n_b16 = (n + 15) >> 4;
  // 32-bit divisions (w < 1024 workgroups, < 2^21 blocks): a 64-bit one is a long instruction sequence on the GPU
  const int b_lo = (int)((unsigned)w * (unsigned)n_b16 / (unsigned)gs);
  const int nb = (int)((unsigned)(w + 1) * (unsigned)n_b16 / (unsigned)gs) - b_lo;
  const int ldy = AK_PICK(sg, sgs.ldy);
  uint16_t* const yseg = AK_PICK(sg, sgs.y) + (TH ? (size_t)th * 8 * ldy : 0);
  float* spart = a.part + (TH ? (size_t)th * P * MP * n_b16 * 16 : 0);
  int* scnt = a.cnt + (TH ? th * (thw / P) : 0);
  if constexpr (SK) {
#pragma unroll
    for (int i = 0; i < kMaxSegs - 1; ++i)
      if (i < sg) spart += (size_t)P * MP * ((AK_PICK(i, sgs.n) + 15) >> 4) * 16;
    scnt += wg0 / P + r;
  }
  // the segment's stripe partials as a buffer (below 2 GB: P x tokens x rows x 4 B)
  const __amdgpu_buffer_rsrc_t rpart = __builtin_amdgcn_make_buffer_rsrc(spart, (short)0, 0x7FFFFFFF, kRsrcWord3);
  (void)rpart;

  // chunks of stripes and the groups an activation image holds (the largest chunk's)
  const int nch = CH ? a.nb : 1;
  int cgs = ngroups;
  if constexpr (SK) cgs = 4 * (stripe_begin(psk + 1, nquad, P, 2) - stripe_begin(psk, nquad, P, 2));
  if constexpr (CH) {
    cgs = 0;
    for (int q = 0; q < nch; ++q) {
      const int gq = 4 * (stripe_begin((q + 1) * P / nch, nquad, P, 2) - stripe_begin(q * P / nch, nquad, P, 2));
      cgs = gq > cgs ? gq : cgs;
    }
  }

  // LDS: zeros [256 B] | A image [group][half][token group][chunk][4 tokens x 3 limbs x 16 B] |
  //      meta [token group][group][4 tokens] int4 | outputs [nb][MP][16] bf16 | partials [nb][P][MP][16] | tickets
  uint8_t* const ximg = lds + 256;
  const int abytes = mt_a_bytes(cgs, NT);
  i32x4* const meta = reinterpret_cast<i32x4*>(ximg + abytes);
  uint16_t* const yl = reinterpret_cast<uint16_t*>(ximg + abytes + mt_meta_bytes(cgs, NT));
  float* const part = reinterpret_cast<float*>(yl + nb * MP * 16);
  int* const tickets = reinterpret_cast<int*>(part + (SPLIT > 1 || CH ? nb * P * MP * 16 : 0));

  if (SPLIT > 1)
    for (int i = tid; i < nb; i += 64 * nwv) tickets[i] = 0;
  if (tid < 64) reinterpret_cast<uint32_t*>(lds)[tid] = 0u;

  // one chunk (an unchunked launch calls it once, outside any loop: a one-trip loop around the item loop makes the
  // compiler spill)
  auto run_chunk = [&](int ch) {
  // chunked: an opaque thread index per chunk, so that nothing lane-dependent is hoisted out of the chunk loop (the
  // hoisted values would stay live across every chunk's item loop)
  int tidc = tid;
  if constexpr (CH) asm volatile("" : "+v"(tidc));
  const int lane = tidc & 63, c = lane & 15, h = lane >> 4;
  // this chunk: stripes [cpa, cpb), groups [g0, g0 + cg) (the whole k unless CH)
  const int cpa = CH ? ch * P / nch : SK ? psk : 0, cpb = CH ? (ch + 1) * P / nch : SK ? psk + 1 : P;
  const int g0 = CH || SK ? 4 * stripe_begin(cpa, nquad, P, 2) : 0;
  const int cg = CH || SK ? 4 * stripe_begin(cpb, nquad, P, 2) - g0 : ngroups;

  // ---- activations, step 1: this lane's bf16 inputs (unit u = (token u / cg, group g0 + u % cg)), requested and
  // waited for before any weight request
  const int sub = lane % LPU, units = cg * mm, ustride = nwv * UPW;  // real tokens only (padding rows unused)
  const int u0 = wave * UPW + lane / LPU;
  const int npass = (units + ustride - 1) / ustride;
  uint4 xv[XB];
  // chained: x (the step's activations, mm x k) read device-coherently, or its tagged copy a.xtg (the same layout in
  // 32-bit words) polled until every word the wave holds carries the launch's tag
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(xb), (short)0, mm * k * 2, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rxt =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(a.xtg), (short)0, mm * k * 4, kRsrcWord3);
  const bool tagged = CHAIN && a.xtg != nullptr;
  const uint32_t tag2 = (tag & kMtTagMask) * 0x10001u;
  (void)rx, (void)rxt, (void)tag2;
  auto ld_coherent = [&](int o) __attribute__((always_inline)) {
    if constexpr (BITS == 4) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, (o + unit_pair_offset<4>(sub, 0)) * 2, 0, kSc1);
      return make_uint4(v[0], v[1], v[2], v[3]);
    } else {
      uint32_t v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[q] = __builtin_amdgcn_raw_buffer_load_b32(rx, (o + unit_pair_offset<BITS>(sub, q)) * 2, 0, kSc1);
      return make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  // the lane's pairs of the unit at element offset o from the tagged copy (device-coherent): whether all carry the tag
  auto ld_tagged = [&](int o, uint4& v) __attribute__((always_inline)) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    uint32_t lo[4], hi[4];
    if constexpr (BITS == 4) {
      const int bo = (o + unit_pair_offset<4>(sub, 0)) * 4;
      const u32x4 d0 = __builtin_amdgcn_raw_buffer_load_b128(rxt, bo, 0, kSc1);
      const u32x4 d1 = __builtin_amdgcn_raw_buffer_load_b128(rxt, bo + 16, 0, kSc1);
      lo[0] = d0[0], hi[0] = d0[1], lo[1] = d0[2], hi[1] = d0[3];
      lo[2] = d1[0], hi[2] = d1[1], lo[3] = d1[2], hi[3] = d1[3];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x2 d = __builtin_amdgcn_raw_buffer_load_b64(rxt, (o + unit_pair_offset<BITS>(sub, q)) * 4, 0, kSc1);
        lo[q] = d[0], hi[q] = d[1];
      }
    }
    bool ok = true;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      w[q] = __builtin_amdgcn_perm(hi[q], lo[q], 0x05040100u);              // the two values
      ok = ok && __builtin_amdgcn_perm(hi[q], lo[q], 0x07060302u) == tag2;  // the two tags
    }
    v = make_uint4(w[0], w[1], w[2], w[3]);
    return ok;
  };
  auto xload = [&](int pass0) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      const int u = u0 + (pass0 + b) * ustride, t = u / cg, gk = (g0 + u - t * cg) * kG;
      const bool ok = u < units && t < mm && gk < k;
      xv[b] = make_uint4(0u, 0u, 0u, 0u);
      if (pass0 + b < npass) {
        const size_t xo = ok ? (size_t)t * (ACT ? 2 * k : k) + gk : 0;  // the unit's group
        if constexpr (CHAIN) {
          if (tagged) {
            if (wave * UPW + (pass0 + b) * ustride >= units) continue;  // no unit of this wave in the pass (uniform)
            const long long t0 = wall_clock64();
            for (;;) {
              uint4 v;
              const bool got = ld_tagged((int)xo, v);
              if (__all(got || !ok)) {
                xv[b] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
                break;
              }
              if (wall_clock64() - t0 > kMtChainSpinTicks) {
                if (lane == 0) __hip_atomic_store(&g_mt_chain_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
              }
              __builtin_amdgcn_s_sleep(1);
            }
          } else {
            const uint4 v = ld_coherent((int)xo);
            xv[b] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
          }
        } else {
          uint4 v = load_unit<BITS>(xb + xo, sub);
          if constexpr (ACT) v = silu_mul8(v, load_unit<BITS>(xb + xo + k, sub));
          xv[b] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
  };
  if constexpr (!CHAIN) {
    xload(0);
#pragma unroll
    for (int b = 0; b < XB; ++b) asm volatile("" ::"v"(xv[b].x), "v"(xv[b].y), "v"(xv[b].z), "v"(xv[b].w));
  }

  // ---- this wave's tasks: stripe set j, quads [qa, qb), blocks b0w, b0w + bstep, ... < nb
  const int j = wave % SPLIT, bstep = nwv / SPLIT, b0w = wave / SPLIT;
  const int pa = CH || SK ? cpa : j * P / SPLIT, pb = CH || SK ? cpb : (j + 1) * P / SPLIT;
  const int qa = stripe_begin(pa, nquad, P, 2), qb = stripe_begin(pb, nquad, P, 2);
  const int ntw = b0w < nb ? (nb - b0w + bstep - 1) / bstep : 0;
  const int nitems = ntw * (qb - qa);
  // bit q - qa set when quad q is the last of its stripe (quads < qa + 128)
  unsigned long long ends0 = 0, ends1 = 0;
  for (int p = pa; p < pb; ++p) {
    const int r = stripe_begin(p + 1, nquad, P, 2) - 1 - qa;
    if (r < 64) ends0 |= 1ull << r;
    else ends1 |= 1ull << (r - 64);
  }

  // ---- weight addressing: per lane fixed, per item scalar.  Rows past the segment's end (padding of the last block)
  // read other rows or, past the buffer, zeros; their results are not written.
  const int ntile = nquad >> 1;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(AK_PICK(sg, sgs.wt)), (short)0, ntile * n * REC, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(AK_PICK(sg, sgs.st)), (short)0, ntile * n * 16, kRsrcWord3);
  // pair loads (quad_vo_w / quad_vo_h): load e reads row 2 (c >> 1) + e, the even lane of a column pair the first half
  // of each line, the odd lane the second; W2 / W3 after quad_pair_rows: the chunk pair 2 (h >> 1), 2 (h >> 1) + 1 of
  // group 2 jj + (h & 1) in lo[jj]
  const int vo_w = quad_vo_w(BITS, c, h, REC), vo_h = quad_vo_h(c, h, REC), vo_s = c * 16;
  const int tile_w = n * REC, tile_s = n * 16;
  auto fetch1 = [&](int blk, int qd, QuadRaw<BITS>& d) {
    const int row0 = (b_lo + blk) * 16, odd = qd & 1;
    const int so = row0 * REC + (qd >> 1) * tile_w;
    if constexpr (BITS == 4) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {  // line s >> 1 of row 2 (c >> 1) + (s & 1)
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, so + odd * 256 + (s >> 1) * 128 + (s & 1) * REC, kNt);
        d.w[s] = make_uint4(v[0], v[1], v[2], v[3]);
      }
    } else {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, so + odd * 128 + jj * REC, kNt);
        d.lo[jj] = make_uint4(v[0], v[1], v[2], v[3]);
        if constexpr (BITS == 3) {
          typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 g2 = __builtin_amdgcn_raw_buffer_load_b64(rw, vo_h, so + odd * 64 + jj * REC, kNt);
          d.hi[jj] = make_uint2(g2[0], g2[1]);
        }
      }
    }
    typedef unsigned int u32x2s __attribute__((ext_vector_type(2)));
    const u32x2s sv = __builtin_amdgcn_raw_buffer_load_b64(rs, vo_s, row0 * 16 + (qd >> 1) * tile_s + odd * 8, 0);
    d.s = make_uint2(sv[0], sv[1]);
  };

  QuadRaw<BITS> buf[DEPTH];
  // fetch cursor (an item past the end reloads quad qa of block 0: cache-resident, never used)
  int fb = b0w, fq = qa;
  auto fetch_next = [&](QuadRaw<BITS>& dst) {
    const bool in = fb < nb;
    fetch1(in ? fb : 0, in ? fq : qa, dst);
    const bool wrap = fq + 1 == qb;
    fq = wrap ? qa : fq + 1;
    fb = wrap ? fb + bstep : fb;
  };
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) fetch_next(buf[d]);
  if constexpr (CHAIN) {  // the first weights are requested: now the wait and the activations
    if (wait && wave == 0) mt_chain_poll(target);
    if (wait) mt_lds_barrier();
    xload(0);
  }

  // ---- activations, step 2: limbs into the A image, bias sums and activation scale into meta
  auto convert = [&](int p0) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      if (p0 + b >= npass || wave * UPW + (p0 + b) * ustride >= units) break;  // no unit of this wave (uniform)
      const int u = u0 + (p0 + b) * ustride;
      const bool live = u < units;
      const int t = live ? u / cg : 0, g = live ? u - t * cg : 0, tg = t >> 2, ui = t & 3;  // g: of the chunk
      const int eg0 = 8 * sub, ch = eg0 >> 5;
      int b0, b1, b2;
      const int e = convert_unit<BITS>(xv[b], ximg + ((g * 2) * NT + tg) * 768 + ch * 192 + ui * 48, NT * 768,
                                       sub & 3, live, b0, b1, b2);
      if (live) {
        if (sub == 0) {
          constexpr int OFF = code_offset<BITS>();
          const i32x4 mv = {-OFF * b0, -OFF * b1, -OFF * b2, act_scale_bits(e)};
          meta[(tg * cgs + g) * 4 + ui] = mv;
        }
      }
    }
  };
  convert(0);
  for (int p0 = XB; p0 < npass; p0 += XB) {
    xload(p0);
    convert(p0);
  }
  __syncthreads();

  // A role: token (c >> 2) of the token group, limb c & 3 (limb 3 reads zeros at the pass's 4 free bank slots)
  const bool a_on = (c & 3) < 3;
  const int a_lane = a_on ? 256 + h * 192 + 16 * (3 * (c >> 2) + (c & 3)) : 16 * ((12 * h + 12 + (c >> 2)) & 15);
  const int a_gmul = a_on ? 2 * NT * 768 : 0, a_hmul = a_on ? NT * 768 : 0, a_tmul = a_on ? 768 : 0;

  auto write_y = [&](int bl, int tg, float y) {  // row c of local block bl, token 4 tg + h
    yl[(bl * MP + 4 * tg + h) * 16 + c] = f2bf(y);
  };

  int cb = b0w, cq = qa, cpp = pa;
  float acc[NT][4], yrun[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    yrun[t] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[t][s] = 0.f;
  }
  // one item without branches: an[][] = the accumulators before a stripe end reset them
  auto core = [&](QuadRaw<BITS>& bf, float (&an)[NT][4], bool& end, int& eg, int& ep) {
    const int r0 = cq - qa;
    end = ((r0 < 64 ? ends0 >> r0 : ends1 >> (r0 - 64)) & 1ull) != 0;
    // scales first: the loaded dwords die here (scales live to the end of the item would be copied at the loop latch)
    float sc[4];
    sc[0] = __uint_as_float(bf.s.x << 16);
    sc[1] = __uint_as_float(bf.s.x & 0xFFFF0000u);
    sc[2] = __uint_as_float(bf.s.y << 16);
    sc[3] = __uint_as_float(bf.s.y & 0xFFFF0000u);
    asm volatile("" ::"v"(sc[0]), "v"(sc[1]), "v"(sc[2]), "v"(sc[3]));
    quad_pair_rows<BITS>(bf, (c & 1) != 0);  // in place: the buffer is refilled after the item
    Raw<BITS> rq[4];
    quad_groups<BITS>(bf, rq);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      i32x4 b0, b1;
      make_b<BITS>(rq[s], b0, b1);
      const int g = 4 * cq + s - g0;  // group of the chunk's image
#pragma unroll
      for (int tg = 0; tg < NT; ++tg) {
        if constexpr (NT > 2) asm volatile("" ::: "memory");  // one token group's operands live at a time
        const i32x4 mt = meta[(tg * cgs + g) * 4 + h];
        const uint8_t* src = lds + a_lane + g * a_gmul + tg * a_tmul;
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(src);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(src + a_hmul);
        i32x4 d = mt;
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
        acc[tg][s] = fmaf(group_sum_f32(d), sc[s] * __int_as_float(mt[3]), acc[tg][s]);
      }
    }
#pragma unroll
    for (int tg = 0; tg < NT; ++tg)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        an[tg][s] = acc[tg][s];
        acc[tg][s] = end ? 0.f : acc[tg][s];
      }
    eg = cb;
    ep = cpp;
    cpp = end ? cpp + 1 : cpp;
    const bool wrap = cq + 1 == qb;
    cq = wrap ? qa : cq + 1;
    cb = wrap ? cb + bstep : cb;
    cpp = wrap ? pa : cpp;
  };
  // a stripe ended: its partial per (row, token) = ((slot 0 + slot 1) + slot 2) + slot 3 in the lane
  auto stripe_end = [&](const float (&v)[NT][4], int eg, int ep) {
    float pp[NT];
#pragma unroll
    for (int tg = 0; tg < NT; ++tg) pp[tg] = ((v[tg][0] + v[tg][1]) + v[tg][2]) + v[tg][3];
    if constexpr (CH) {  // added in stripe order after the last chunk
#pragma unroll
      for (int tg = 0; tg < NT; ++tg) part[((eg * P + ep) * MP + 4 * tg + h) * 16 + c] = pp[tg];
    } else if constexpr (SK) {  // to the range's partials, device-coherent (the range's last workgroup adds them)
      // (block-major: [stripe][block][token][row]; a buffer store with the block's offset scalar and the lane's part a
      // per-lane constant, device-coherent as an agent-scope atomic store)
      const int so = ((ep * n_b16 + b_lo + eg) * MP * 16) * 4;
#pragma unroll
      for (int tg = 0; tg < NT; ++tg)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pp[tg]), rpart, ((4 * tg + h) * 16 + c) * 4, so, kSc1);
    } else if constexpr (SPLIT == 1) {
#pragma unroll
      for (int tg = 0; tg < NT; ++tg) {
        yrun[tg] = ep == 0 ? pp[tg] : yrun[tg] + pp[tg];
        if (ep == P - 1) write_y(eg, tg, yrun[tg]);
      }
    } else {
#pragma unroll
      for (int tg = 0; tg < NT; ++tg) part[((eg * P + ep) * MP + 4 * tg + h) * 16 + c] = pp[tg];
      if (ep + 1 < pb) return;  // more stripes in this task
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  // LDS only: no wait for loads in flight
      int last = 0;
      if (lane == 0) last = atomicAdd(&tickets[eg], 1) == SPLIT - 1;
      last = __shfl(last, 0);
      if (last) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        const float* slot = part + eg * P * MP * 16;
#pragma unroll
        for (int tg = 0; tg < NT; ++tg) {
          const int o = (4 * tg + h) * 16 + c;
          float y = slot[o];
          for (int q = 1; q < P; ++q) y += slot[q * MP * 16 + o];
          write_y(eg, tg, y);
        }
      }
    }
  };

  const int nfull = nitems / DEPTH * DEPTH;
  for (int i0 = 0; i0 < nfull; i0 += DEPTH) {
    float sv[DEPTH][NT][4];
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
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    if (nfull + d < nitems) {
      float v[NT][4];
      bool e;
      int g, p;
      core(buf[d], v, e, g, p);
      if (e) stripe_end(v, g, p);
    }
  }
  if constexpr (CH) __syncthreads();  // the chunk's image is free, its partials are in
  };
  if constexpr (CH) {
    for (int ch = 0; ch < nch; ++ch) run_chunk(ch);
  } else {
    run_chunk(0);
  }
  if constexpr (SK) {
    // every wave's partial stores are acknowledged at device scope before the range's counter moves
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    int* const last = reinterpret_cast<int*>(yl);
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(scnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last = old == P - 1;
      if (old == P - 1) __hip_atomic_store(scnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
    }
    __syncthreads();
    if (!*last) return;
    __syncthreads();  // every thread has read the flag before the outputs overwrite it
    // two outputs per thread at a time (their partials' loads in flight together; block-major partials: the
    // workgroup's outputs are the contiguous run from b_lo * MP * 16, in yl's order)
    // (two token groups: one at a time, as two spill the W2 kernel's registers)
    const int ne = nb * MP * 16, st = 64 * nwv;
    if constexpr (NT == 2) {
      for (int i = tid; i < ne; i += st)
        yl[i] = f2bf(sum_stripe_partials(spart, (size_t)b_lo * MP * 16 + i, (size_t)MP * n_b16 * 16, P));
    } else {
      for (int i0 = tid; i0 < ne; i0 += 2 * st) {
        const size_t o0 = (size_t)b_lo * MP * 16 + i0, o1 = (size_t)b_lo * MP * 16 + (i0 + st < ne ? i0 + st : i0);
        const size_t off[2] = {o0, o1};
        float y[2];
        sum_stripe_partials_n<2>(spart, off, (size_t)MP * n_b16 * 16, P, y);
        yl[i0] = f2bf(y[0]);
        if (i0 + st < ne) yl[i0 + st] = f2bf(y[1]);
      }
    }
  }
  if constexpr (CH) {
    for (int i = tid; i < nb * MP * 16; i += 64 * nwv) {
      const int bl = i / (MP * 16), o = i - bl * MP * 16;
      const float* slot = part + bl * P * MP * 16;
      float y = slot[o];
      for (int q = 1; q < P; ++q) y += slot[q * MP * 16 + o];
      yl[i] = f2bf(y);
    }
  }
  __syncthreads();
  uint32_t* const ytg = CHAIN ? AK_PICK(sg, a.ytg) : nullptr;
  for (int i = tid; i < nb * MP * 16; i += 64 * nwv) {
    const int bl = i / (MP * 16), t = (i / 16) % MP, row = (b_lo + bl) * 16 + (i & 15);
    if (t < mm && row < n) {
      if constexpr (CHAIN) {
        __hip_atomic_store(yseg + (size_t)t * ldy + row, yl[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ytg)
          __hip_atomic_store(ytg + (size_t)t * ldy + row, (uint32_t)yl[i] | ((tag & kMtTagMask) << 16),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        yseg[(size_t)t * ldy + row] = yl[i];
      }
    }
  }
}

template <int BITS, int SPLIT, int DEPTH, int NT, bool CH, bool SK = false, bool ACT = false, bool TH = false>
__global__ void __launch_bounds__(1024, 1) i8_mt_kernel(const I8Args a) {
  extern __shared__ __attribute__((aligned(256))) uint8_t lds[];
  mt_body<BITS, SPLIT, DEPTH, NT, CH, SK, ACT, TH>(a, lds, false, 0u, 0u);
}

size_t mt_block_bytes(int P, int split, int nt) {  // per 16-row block: outputs, partials, ticket
  return (size_t)4 * nt * 16 * 2 + (split > 1 ? (size_t)P * 4 * nt * 16 * 4 + 4 : 0);
}

template <int BITS, int SPLIT, int NT, bool CH, bool SK = false, bool ACT = false, bool TH = false>
void launch_mt_split(const I8Args& a, int grid, size_t smem, hipStream_t s) {
  constexpr int DEPTH = NT > 2 ? 1 : 2;  // items in flight per wave (16 tokens: their accumulators take the registers)
  hipLaunchKernelGGL((i8_mt_kernel<BITS, SPLIT, DEPTH, NT, CH, SK, ACT, TH>), dim3(grid), dim3(1024), smem, s, a);
}

// groups of the largest of nch chunks of stripes
int mt_chunk_groups(int nquad, int P, int nch) {
  int cg = 0;
  for (int q = 0; q < nch; ++q) {
    const int gq = 4 * (stripe_begin((q + 1) * P / nch, nquad, P, 2) - stripe_begin(q * P / nch, nquad, P, 2));
    cg = gq > cg ? gq : cg;
  }
  return cg;
}

// split-K for activations beyond the LDS up to this many 16-row blocks per CU.  Measured at 16 tokens, k = 5120:
// gate_up (13.5 blocks per CU) 55-64 -> 44-57 us and the 152064-row LM head (37 per CU, two 8-token launches before)
// 167 -> 145 us against the chunked launch; the stripe partials (P x tokens x rows x 4 B) stay well below the weights.
#ifndef AK_MT_SK_BLOCKS
#define AK_MT_SK_BLOCKS 40
#endif
template <int BITS, int NT>
int launch_mt(I8Args a, hipStream_t s) {
  const Segs& g = a.segs;
  const int ngroups = a.nquad * 4, ntile = a.nquad / 2;
  for (int i = 0; i < g.nseg; ++i)  // buffer offsets are 32-bit
    if ((long long)ntile * g.n[i] * 128 * BITS >= (1ll << 31)) return AK_INVALID;
  // workgroups per segment: about the same number of 16-row blocks each, at most one workgroup per CU
  int total = 0;
  for (int i = 0; i < g.nseg; ++i) total += (g.n[i] + 15) / 16;
  const int cus = num_cus();
  int per = (total + cus - 1) / cus, grid = 0;
  for (;; ++per) {
    grid = 0;
    for (int i = 0; i < g.nseg; ++i) grid += ((g.n[i] + 15) / 16 + per - 1) / per;
    if (grid <= cus || per >= total) break;
  }
  for (int i = 0, e = 0; i < kMaxSegs; ++i) {
    if (i < g.nseg) e += ((g.n[i] + 15) / 16 + per - 1) / per;
    a.wg_end[i] = e;
  }
  int nbmax = 0;
  for (int i = 0; i < g.nseg; ++i) {
    const int nbs = (g.n[i] + 15) / 16, gs = (nbs + per - 1) / per;
    nbmax = (nbs + gs - 1) / gs > nbmax ? (nbs + gs - 1) / gs : nbmax;
  }
  // split-K across workgroups: P workgroups per row range, each one stripe, partials in the stream's scratch; taken
  // when the launch has few rows per CU (every workgroup would convert all of x for at most two 16-row blocks), or
  // when the activation image does not fit the LDS and there are not many rows per CU.  Row ranges are shared out over the segments by their blocks.
  // Without scratch (inside a capture that has not got it yet): the launches below.
  const size_t x_bytes = 256 + (size_t)mt_a_bytes(ngroups, NT) + mt_meta_bytes(ngroups, NT);
  if (a.P >= 2 && (total <= 2 * cus || (x_bytes > 140 * 1024 && total <= AK_MT_SK_BLOCKS * cus))) {
    const int nrt = cus / a.P;
    int nr[kMaxSegs] = {0, 0, 0, 0}, left = nrt - g.nseg, nbr = 0;
    size_t part_floats = 0;
    for (int i = 0; i < g.nseg; ++i) {  // at least one range per segment, the rest by blocks
      const int nbs = (g.n[i] + 15) / 16;
      nr[i] = 1 + (int)((long long)left * nbs / total);
      nbr = (nbs + nr[i] - 1) / nr[i] > nbr ? (nbs + nr[i] - 1) / nr[i] : nbr;
      part_floats += (size_t)a.P * 4 * NT * nbs * 16;
    }
    const int cg = mt_chunk_groups(a.nquad, a.P, a.P);
    const size_t smem = 256 + (size_t)mt_a_bytes(cg, NT) + mt_meta_bytes(cg, NT) + (size_t)nbr * 4 * NT * 16 * 2 + 16;
    void* z = nrt >= g.nseg && nrt <= 1024 && smem <= 160 * 1024 ? stream_scratch(s, 4096 + part_floats * 4) : nullptr;
    if (z) {
      I8Args b = a;
      for (int i = 0, e = 0; i < kMaxSegs; ++i) {
        if (i < g.nseg) e += nr[i] * a.P;
        b.wg_end[i] = e;
      }
      b.cnt = static_cast<int*>(z);
      b.part = reinterpret_cast<float*>(static_cast<uint8_t*>(z) + 4096);
      if (a.act)
        launch_mt_split<BITS, 1, NT, false, true, true>(b, b.wg_end[g.nseg - 1], smem, s);
      else
        launch_mt_split<BITS, 1, NT, false, true>(b, b.wg_end[g.nseg - 1], smem, s);
      return (int)hipGetLastError();
    }
    // 9..16 tokens, one segment, one stripe's 16-token image beyond the LDS: both 8-token halves in one split-K
    // launch (NT = 2 each, the same results as two 8-token launches).  Half the row ranges per half keep the grid at
    // one workgroup per CU, and the two halves of a (range, stripe) run at once on the same XCD (workgroups nrh * P apart),
    // so the second one's weights come from the L2: down 5120 x 27648 at 16 tokens, W2 / W3 / W4 44.8 / 59.6 / 54.4 ->
    // 30.4 / 42.9 / 40.7 us (full ranges per half, two rounds of workgroups: 43.3 / 57.1 / 52.5 us).
    if constexpr (NT == 4) {
      // row ranges per half, a multiple of 8 / gcd(P, 8) so that nrh * P is a multiple of the 8 XCDs (workgroup i runs
      // on XCD i % 8: the two halves of a (range, stripe), nrh * P workgroups apart, then share an XCD's L2)
      const int xq = 8 / (a.P % 8 == 0 ? 8 : a.P % 4 == 0 ? 4 : a.P % 2 == 0 ? 2 : 1);
      const int nrh = nrt / 2 / xq * xq > 0 ? nrt / 2 / xq * xq : xq;
      const int nbs = (g.n[0] + 15) / 16, nbr2 = (nbs + nrh - 1) / nrh;
      const size_t smem2 = 256 + (size_t)mt_a_bytes(cg, 2) + mt_meta_bytes(cg, 2) + (size_t)nbr2 * 4 * 2 * 16 * 2 + 16;
      const size_t pf = (size_t)a.P * 4 * 2 * nbs * 16;  // one half's stripe partials (floats)
      if (g.nseg == 1 && a.m > 8 && 2 * nrh <= 1024 && smem2 <= 160 * 1024) {
        void* z2 = stream_scratch(s, 4096 + 2 * pf * 4);
        if (z2) {
          I8Args b = a;
          for (int i = 0; i < kMaxSegs; ++i) b.wg_end[i] = nrh * a.P;
          b.cnt = static_cast<int*>(z2);
          b.part = reinterpret_cast<float*>(static_cast<uint8_t*>(z2) + 4096);
          if (a.act)
            launch_mt_split<BITS, 1, 2, false, true, true, true>(b, 2 * nrh * a.P, smem2, s);
          else
            launch_mt_split<BITS, 1, 2, false, true, false, true>(b, 2 * nrh * a.P, smem2, s);
          return (int)hipGetLastError();
        }
      }
    }
  }
  if (a.act) return AK_INVALID;  // the SiLU(gate) * up activation: split-K launches only (the caller falls back)
  if (x_bytes <= 140 * 1024) {
    // the whole activation image fits: tasks per block = fewest quad rounds for the busiest wave, a task's overhead
    // counted as about one quad
    int best_split = 1;
    double best = 1e30;
    for (int split : {1, 2, 4, 8}) {
      if (split > a.P) break;
      if (x_bytes + (size_t)nbmax * mt_block_bytes(a.P, split, NT) + 16 > 160 * 1024) continue;
      int lmax = 0;
      for (int j = 0; j < split; ++j) {
        const int l = stripe_begin((j + 1) * a.P / split, a.nquad, a.P, 2) - stripe_begin(j * a.P / split, a.nquad, a.P, 2);
        lmax = l > lmax ? l : lmax;
      }
      const int bstep = 16 / split;
      const double cost = (double)((nbmax + bstep - 1) / bstep) * (lmax + 1.0);
      if (cost < best - 1e-9) best = cost, best_split = split;
    }
    if (best < 1e29) {
      const size_t smem = x_bytes + (size_t)nbmax * mt_block_bytes(a.P, best_split, NT) + 16;
      switch (best_split) {
        case 1: launch_mt_split<BITS, 1, NT, false>(a, grid, smem, s); break;
        case 2: launch_mt_split<BITS, 2, NT, false>(a, grid, smem, s); break;
        case 4: launch_mt_split<BITS, 4, NT, false>(a, grid, smem, s); break;
        default: launch_mt_split<BITS, 8, NT, false>(a, grid, smem, s); break;
      }
      return (int)hipGetLastError();
    }
  }
  // chunked: the fewest chunks of stripes whose image, with every block's stripe partials, fits the LDS
  const size_t blk = (size_t)4 * NT * 16 * 2 + (size_t)a.P * 4 * NT * 16 * 4;
  for (int nch = 2; nch <= a.P; ++nch) {
    const int cg = mt_chunk_groups(a.nquad, a.P, nch);
    const size_t smem = 256 + (size_t)mt_a_bytes(cg, NT) + mt_meta_bytes(cg, NT) + (size_t)nbmax * blk + 16;
    if (smem > 160 * 1024) continue;
    a.nb = nch;
    launch_mt_split<BITS, 1, NT, true>(a, grid, smem, s);
    return (int)hipGetLastError();
  }
  return AK_INVALID;
}

// ---- chained launches (3..4 tokens)
constexpr int kMtSplitK = 256;
struct MtChainStep {
  I8Args a;
  int kind;    // bits * 16 + SPLIT (whole activation image), + kMtSplitK for a split-K step (SPLIT 1)
  int wait;    // 1: the step reads (or overwrites) what earlier steps wrote or read: the grid barrier
  int signal;  // 1: a later step waits at the grid barrier for this one: the flags move after it
};

// epochs: one word per workgroup, the launches of this chain so far (the tag of a launch: the low 16 bits of its
// epoch + 1, which differ from the previous launch's tags and from the initial zeros)
template <int NT>
__global__ void __launch_bounds__(1024, 1) i8_mt_chain_kernel(const MtChainStep* __restrict__ steps, int nsteps,
                                                              uint32_t* __restrict__ epochs) {
  extern __shared__ __attribute__((aligned(256))) uint8_t lds[];
  constexpr int D = NT > 2 ? 1 : 2;
  uint32_t* const flag = g_mt_chain_flags + blockIdx.x;
  // every workgroup's flag holds the same count between chained launches (all of them signal the last step)
  const uint32_t f0 =
      __builtin_amdgcn_readfirstlane(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const uint32_t ep = __builtin_amdgcn_readfirstlane(epochs[blockIdx.x]);
  const uint32_t tag = (ep + 1u) & kMtTagMask;
  for (int s = 0; s < nsteps; ++s) {
    const MtChainStep st = steps[s];
    const bool w = st.wait != 0;
    const uint32_t target = f0 + (uint32_t)s;
    switch (st.kind) {
      case 4 * 16 + 1: mt_body<4, 1, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 4 * 16 + 2: mt_body<4, 2, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 4 * 16 + 4: mt_body<4, 4, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 4 * 16 + 8: mt_body<4, 8, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 3 * 16 + 1: mt_body<3, 1, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 3 * 16 + 2: mt_body<3, 2, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 3 * 16 + 4: mt_body<3, 4, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 3 * 16 + 8: mt_body<3, 8, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 2 * 16 + 2: mt_body<2, 2, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 2 * 16 + 4: mt_body<2, 4, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case 2 * 16 + 8: mt_body<2, 8, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;
      case kMtSplitK + 4 * 16 + 1: mt_body<4, 1, D, NT, false, true, false, false, true>(st.a, lds, w, target, tag); break;
      case kMtSplitK + 3 * 16 + 1: mt_body<3, 1, D, NT, false, true, false, false, true>(st.a, lds, w, target, tag); break;
      case kMtSplitK + 2 * 16 + 1: mt_body<2, 1, D, NT, false, true, false, false, true>(st.a, lds, w, target, tag); break;
      default: mt_body<2, 1, D, NT, false, false, false, false, true>(st.a, lds, w, target, tag); break;  // W2, 1
    }
    // signal: this workgroup's outputs of steps <= s are stored (each wave waits for its stores' acknowledgement,
    // which for device-coherent stores means written through); otherwise the workgroup goes on at once
    if (st.signal || s + 1 == nsteps) {
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      __syncthreads();
      if (threadIdx.x == 0) __hip_atomic_store(flag, f0 + (uint32_t)s + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      mt_lds_barrier();
    }
  }
  if (threadIdx.x == 0) epochs[blockIdx.x] = ep + 1u;
}

// The launch shape of one chained step (the choices of launch_mt without its chunked and token-halves forms): 0 with
// a.wg_end, *kind, *smem and *scratch (bytes of counters and stripe partials, split-K only) set; AK_INVALID if the
// step needs a form the chained kernel does not run.
int mt_chain_plan(I8Args& a, int bits, int nt, int* kind, size_t* smem, size_t* scratch) {
  const Segs& g = a.segs;
  const int ngroups = a.nquad * 4, ntile = a.nquad / 2;
  for (int i = 0; i < g.nseg; ++i)
    if ((long long)ntile * g.n[i] * 128 * bits >= (1ll << 31)) return AK_INVALID;
  int total = 0;
  for (int i = 0; i < g.nseg; ++i) total += (g.n[i] + 15) / 16;
  const int cus = num_cus();
  int per = (total + cus - 1) / cus, grid = 0;
  for (;; ++per) {
    grid = 0;
    for (int i = 0; i < g.nseg; ++i) grid += ((g.n[i] + 15) / 16 + per - 1) / per;
    if (grid <= cus || per >= total) break;
  }
  if (grid > cus) return AK_INVALID;
  for (int i = 0, e = 0; i < kMaxSegs; ++i) {
    if (i < g.nseg) e += ((g.n[i] + 15) / 16 + per - 1) / per;
    a.wg_end[i] = e;
  }
  int nbmax = 0;
  for (int i = 0; i < g.nseg; ++i) {
    const int nbs = (g.n[i] + 15) / 16, gs = (nbs + per - 1) / per;
    nbmax = (nbs + gs - 1) / gs > nbmax ? (nbs + gs - 1) / gs : nbmax;
  }
  const size_t x_bytes = 256 + (size_t)mt_a_bytes(ngroups, nt) + mt_meta_bytes(ngroups, nt);
  if (a.P >= 2 && (total <= 2 * cus || (x_bytes > 140 * 1024 && total <= AK_MT_SK_BLOCKS * cus))) {
    const int nrt = cus / a.P;
    int nr[kMaxSegs] = {0, 0, 0, 0}, left = nrt - g.nseg, nbr = 0;
    size_t part_floats = 0;
    for (int i = 0; i < g.nseg; ++i) {
      const int nbs = (g.n[i] + 15) / 16;
      nr[i] = 1 + (int)((long long)left * nbs / total);
      nbr = (nbs + nr[i] - 1) / nr[i] > nbr ? (nbs + nr[i] - 1) / nr[i] : nbr;
      part_floats += (size_t)a.P * 4 * nt * nbs * 16;
    }
    const int cg = mt_chunk_groups(a.nquad, a.P, a.P);
    const size_t sm = 256 + (size_t)mt_a_bytes(cg, nt) + mt_meta_bytes(cg, nt) + (size_t)nbr * 4 * nt * 16 * 2 + 16;
    if (nrt < g.nseg || nrt > 1024 || sm > 160 * 1024) return AK_INVALID;
    for (int i = 0, e = 0; i < kMaxSegs; ++i) {
      if (i < g.nseg) e += nr[i] * a.P;
      a.wg_end[i] = e;
    }
    *kind = kMtSplitK + bits * 16 + 1;
    *smem = sm;
    *scratch = 4096 + part_floats * 4;
    return 0;
  }
  if (x_bytes > 140 * 1024) return AK_INVALID;
  int best_split = 0;
  double best = 1e30;
  for (int split : {1, 2, 4, 8}) {
    if (split > a.P) break;
    if (x_bytes + (size_t)nbmax * mt_block_bytes(a.P, split, nt) + 16 > 160 * 1024) continue;
    int lmax = 0;
    for (int j = 0; j < split; ++j) {
      const int l = stripe_begin((j + 1) * a.P / split, a.nquad, a.P, 2) - stripe_begin(j * a.P / split, a.nquad, a.P, 2);
      lmax = l > lmax ? l : lmax;
    }
    const int bstep = 16 / split;
    const double cost = (double)((nbmax + bstep - 1) / bstep) * (lmax + 1.0);
    if (cost < best - 1e-9) best = cost, best_split = split;
  }
  if (!best_split) return AK_INVALID;
  *kind = bits * 16 + best_split;
  *smem = x_bytes + (size_t)nbmax * mt_block_bytes(a.P, best_split, nt) + 16;
  *scratch = 0;
  return 0;
}

}  // namespace

// 1..16 tokens (4, 8 or 16 in the kernel), 16-row blocks (the last one padded); activations beyond the LDS: split-K
// across workgroups or chunks of stripes.  Returns AK_INVALID if the shape does not suit the kernel (group 64, a segment beyond 2 GB, a chunk of
// one stripe beyond the LDS): the caller falls back.  act = 1: x is the merged gate_up [m][2k] and the activations
// are SiLU(gate) * up.
int i8_gemv_mt(int bits, const void* x, int m, const Segs& g, int k, int group, hipStream_t s, int act) {
  if (group != kG || m < 1 || m > 16) return AK_INVALID;
#ifdef AK_NO_MT
  return AK_INVALID;
#endif
  I8Args a;
  a.act = act;
  a.segs = g;
  a.x = static_cast<const uint16_t*>(x);
  a.m = m;
  a.k = k;
  a.nquad = kpad(k) / kG / 4;
  a.qpt = 2;
  a.P = stripe_count(a.nquad, a.qpt);
  a.nb = 0;
  a.part = nullptr;
  a.cnt = nullptr;
  const int nt = m <= 4 ? 1 : m <= 8 ? 2 : 4;
  switch (bits * 10 + nt) {
    case 41: return launch_mt<4, 1>(a, s);
    case 31: return launch_mt<3, 1>(a, s);
    case 21: return launch_mt<2, 1>(a, s);
    case 42: return launch_mt<4, 2>(a, s);
    case 32: return launch_mt<3, 2>(a, s);
    case 22: return launch_mt<2, 2>(a, s);
    case 44: return launch_mt<4, 4>(a, s);
    case 34: return launch_mt<3, 4>(a, s);
    case 24: return launch_mt<2, 4>(a, s);
    default: return AK_INVALID;
  }
}

// A chain of 1..4-token steps (at least one above 2) as one launch of the tokens-in-A-rows kernel's steps: the table of
// steps in device memory (then the workgroups' epochs, the tagged output copies and the split-K steps' counters and
// partials), or AK_INVALID if a step does not suit the chained kernel (the caller runs one launch per step).  Tagged
// waits as in the one-token chain: step i reads a tagged copy of segment j of step i - 1's outputs where that segment
// holds all of its activations (x = its start, rows dense), step i - 1 waited for the step before it (or is the
// first) and step i + 1 waits (or there is none).  *nt_out: the kernel's token groups (1).
int mt_chain_make(int nsteps, const int* bits, const void* const* x, const int* m, const int* k, const Segs* segs,
                  const int* wait, void** table, int* nt_out, size_t* smem_out) {
  // up to 4 tokens (one token group): with two token groups the chained sweep measured slower than one launch per
  // step (M = 8, 64 layers + LM head: 5684-6215 us against 5488-5508 us with step bodies that spill or run one item
  // in flight per wave, 5891 against 5520 us without spills)
  const int nt = 1;
  for (int i = 0; i < nsteps; ++i)
    if (m[i] < 1 || m[i] > 4 || bits[i] < 2 || bits[i] > 4) return AK_INVALID;
  if (num_cus() > kMtChainMaxWg) return AK_INVALID;
  std::vector<MtChainStep> h((size_t)nsteps);
  const size_t table_bytes = ((size_t)nsteps * sizeof(MtChainStep) + 255) & ~(size_t)255;
  size_t total = table_bytes + kMtChainMaxWg * 4, smem = 0;
  std::vector<size_t> zoff((size_t)nsteps, 0), zbytes((size_t)nsteps, 0), toff((size_t)nsteps, 0);
  std::vector<int> tseg((size_t)nsteps, -1);
  const char* ev = getenv("AK_CHAIN_TAGS");
  const bool tags_on = !(ev && atoi(ev) == 0);
  for (int i = 1; i < nsteps && tags_on; ++i) {
    if (!wait[i] || (i > 1 && !wait[i - 1]) || (i + 1 < nsteps && !wait[i + 1])) continue;
    const Segs& p = segs[i - 1];
    for (int j = 0; j < p.nseg; ++j)
      if (p.y[j] == x[i] && p.ldy[j] == p.n[j] && (long long)m[i] * k[i] <= (long long)m[i - 1] * p.n[j]) {
        tseg[(size_t)i] = j;
        toff[(size_t)i] = total;
        total += ((size_t)m[i - 1] * p.n[j] * 4 + 255) & ~(size_t)255;
        break;
      }
  }
  for (int i = 0; i < nsteps; ++i) {
    I8Args& a = h[(size_t)i].a;
    a.segs = segs[i];
    a.x = static_cast<const uint16_t*>(x[i]);
    a.m = m[i];
    a.k = k[i];
    a.nquad = kpad(k[i]) / kG / 4;
    a.qpt = 2;
    a.P = stripe_count(a.nquad, a.qpt);
    a.nb = 0;
    a.part = nullptr;
    a.cnt = nullptr;
    a.act = 0;
    size_t sm = 0, zb = 0;
    if (mt_chain_plan(a, bits[i], nt, &h[(size_t)i].kind, &sm, &zb)) return AK_INVALID;
    h[(size_t)i].wait = i > 0 && wait[i] && tseg[(size_t)i] < 0 ? 1 : 0;
    h[(size_t)i].signal = i + 1 < nsteps && wait[i + 1] && tseg[(size_t)i + 1] < 0 ? 1 : 0;
    smem = sm > smem ? sm : smem;
    if (zb) {
      zoff[(size_t)i] = total;
      zbytes[(size_t)i] = zb;
      total += (zb + 255) & ~(size_t)255;
    }
  }
  void* d = nullptr;
  int e = (int)hipMalloc(&d, total);
  if (!e) e = (int)hipMemset(static_cast<uint8_t*>(d) + table_bytes, 0, total - table_bytes);
  for (int i = 0; i < nsteps && !e; ++i) {
    if (tseg[(size_t)i] >= 0) {
      uint32_t* tb = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(d) + toff[(size_t)i]);
      h[(size_t)i].a.xtg = tb;
      h[(size_t)i - 1].a.ytg[tseg[(size_t)i]] = tb;
    }
    if (zbytes[(size_t)i]) {
      h[(size_t)i].a.cnt = reinterpret_cast<int*>(static_cast<uint8_t*>(d) + zoff[(size_t)i]);
      h[(size_t)i].a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(d) + zoff[(size_t)i] + 4096);
    }
  }
  if (!e) e = (int)hipMemcpy(d, h.data(), (size_t)nsteps * sizeof(MtChainStep), hipMemcpyHostToDevice);
  if (e) {
    if (d) (void)hipFree(d);
    return e == (int)hipErrorOutOfMemory ? AK_OOM : e;
  }
  *table = d;
  *nt_out = nt;
  *smem_out = smem;
  return 0;
}

int mt_chain_launch(const void* table, int nsteps, int nt, size_t smem, hipStream_t s) {
  const MtChainStep* t = static_cast<const MtChainStep*>(table);
  uint32_t* ep = reinterpret_cast<uint32_t*>(const_cast<uint8_t*>(static_cast<const uint8_t*>(table)) +
                                             (((size_t)nsteps * sizeof(MtChainStep) + 255) & ~(size_t)255));
  if (nt != 1) return AK_INVALID;
  hipLaunchKernelGGL(i8_mt_chain_kernel<1>, dim3(num_cus()), dim3(1024), smem, s, t, nsteps, ep);
  return (int)hipGetLastError();
}

// reads and clears the flag a chained launch of these steps raises when a bounded wait ran out
int mt_chain_error(int* err) {
  uint32_t v = 0, z = 0;
  int e = (int)hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_mt_chain_err), sizeof(v), 0, hipMemcpyDeviceToHost);
  if (!e && v) e = (int)hipMemcpyToSymbol(HIP_SYMBOL(g_mt_chain_err), &z, sizeof(z), 0, hipMemcpyHostToDevice);
  *err = (int)v;
  return e;
}

}  // namespace agq
