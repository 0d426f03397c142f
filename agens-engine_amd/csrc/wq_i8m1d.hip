// The default-numerics GEMV for one token (decode, M = 1), group 128, on gfx950: the same exact integer group sums and
// the same fp32 combine order as wq_i8.hip (rows are bit-identical to any-m launches), with an MFMA layout chosen so
// that every weight load instruction reads whole cache lines.
//
// "Diagonal" layout of v_mfma_i32_16x16x64_i8 for a block of 4 output rows and one quad (4 groups = 16 lane chunks):
//   lane (c, h) = (lane % 16, lane / 16);
//   B column c = (row c >> 2 of the block, group c & 3 of the quad): lane (c, h) holds chunk 4 * (c & 3) + h of that
//     row, so the 16 lanes of one row read its 16 consecutive chunks and one load instruction covers 4 rows x 256 B
//     (W4; W2 and the W3 two-bit planes 128 B, the W3 third-bit plane 64 B);
//   A row c = (group c >> 2, limb c & 3): lane (c, h) holds limb c & 3 of the inputs of chunk 4 * (c >> 2) + h
//     (limb 3 is zero);
//   D[4g + j][4r + v] is the limb-j sum of row r with the inputs of group g; only g == v is used ("the diagonal"):
//     lane (c, h) with (c & 3) == h holds group h of row c >> 2 in its accumulators (limbs 0..2).
// The MFMA work per weight is the same as a 16-row layout (13 of 16 A rows or columns are wasted either way), but the
// loads are line-sized (a load pattern of 16-byte pieces 64 bytes apart reaches only about half the HBM bandwidth),
// the A operand has 12 useful rows instead of 3, and row blocks are 4 rows, so work divides evenly over 256 CUs for
// the decode shapes.
//
// Work decomposition: one persistent workgroup per CU owns a contiguous range of 4-row blocks of one segment.  Its
// tasks are (block, stripe set j < SPLIT) pairs: stripe set j = the contiguous stripes [j P / SPLIT, (j + 1) P / SPLIT),
// i.e. a contiguous run of quads, walked in order (the fp32 order of the numerics).  Wave w always takes stripe set
// w % SPLIT, for the blocks w / SPLIT, w / SPLIT + nwv / SPLIT, ...  With SPLIT = 1 a wave owns whole blocks and adds
// the stripe partials itself; otherwise the partials meet in LDS and the last task of a block to finish (LDS ticket)
// adds them in stripe order.
//
// Item pipeline: every wave streams its items (one quad of one block: one buffer load per lane, two for W3, plus one
// for the scales) through DEPTH register buffers.  A group of DEPTH items is one branch-free block of code, so the
// compiler interleaves the unpacking, LDS reads and MFMAs of neighbouring items: the load offsets are a fixed per-lane
// part plus a scalar part of (block, quad), the cursors advance by selects, and a stripe that ends inside the group
// only leaves a copy of its accumulators; the group's epilogue turns those into stripe partials.
#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_i8_common.h"

// phase timestamps for profiling builds (a build that defines them records them; product builds compile nothing)
#ifndef AK_M1_STAMP
#define AK_M1_STAMP(i)
#define AK_M1_STAMP_AFTER(i, v)
#define AK_M1_STAMP_ITEM(i)
#endif

namespace agq {

int num_cus();

namespace {

constexpr int kG = 128, kCPQ = 16;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, dword 3 (CDNA)
constexpr int kNt = 2;                    // streaming (non-temporal) cache policy for the weights

template <int BITS>
struct Rec {
  static constexpr int bytes = 128 * BITS;          // one row's 1024-input tile
  static constexpr int chunk = BITS == 4 ? 16 : 8;  // bytes of a lane chunk (W3: its two-bit planes)
};

// segment field i (i < 4, wave-uniform) by constant-index selects: indexing the kernel-argument arrays dynamically
// makes the compiler hold their address in vector registers
template <typename T>
__device__ __forceinline__ T pick4(int i, T v0, T v1, T v2, T v3) {
  return i == 0 ? v0 : i == 1 ? v1 : i == 2 ? v2 : v3;
}
#define AK_PICK(i, arr) pick4((i), (arr)[0], (arr)[1], (arr)[2], (arr)[3])
static_assert(kMaxSegs == 4, "segment selects cover four segments");

template <int BITS, int SPLIT, int DEPTH, int RB, int MT>
__global__ void __launch_bounds__(1024, 1) i8_m1d_kernel(const I8Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int LPU = kG / 8, UPW = 64 / LPU, XB = 4;
  constexpr int REC = Rec<BITS>::bytes, CHB = Rec<BITS>::chunk;
  const int P = a.P, nquad = a.nquad, k = a.k, mm = a.m;  // mm <= MT tokens (the others are zero, not written)
  const int nwv = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int rr = c >> 2, vv = c & 3;  // B role: row of the block, group of the quad
  const Segs& sgs = a.segs;

  // this workgroup's segment and its blocks [b_lo, b_lo + nb) of that segment
  int sg = 0;
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) sg += (i < sgs.nseg && (int)blockIdx.x >= a.wg_end[i - 1]) ? 1 : 0;
  const int wg0 = sg ? AK_PICK(sg - 1, a.wg_end) : 0, gs = AK_PICK(sg, a.wg_end) - wg0, w = blockIdx.x - wg0;
  const int n = AK_PICK(sg, sgs.n), n_b4 = (n + 3) >> 2;
  const int b_lo = (int)((long long)w * n_b4 / gs);
  const int nb = (int)((long long)(w + 1) * n_b4 / gs) - b_lo;
  uint16_t* const yseg = AK_PICK(sg, sgs.y);
  const int ldy = AK_PICK(sg, sgs.ldy);

  // LDS: zeros [512 B] | limbs [MT][nquad][half 2][chunk 16][limb 3][16 B] | meta [MT][nquad][4] int4 |
  //      outputs [MT][nb][4] bf16 | partials [nb][P][MT][4] | tickets [nb]
  // (48-byte chunk stride: the 12 active lanes of each 16-lane pass of an A read hit 12 distinct 16-byte bank slots of
  // the 256-byte bank row, and the 4 zero-operand lanes read zeros placed in the 4 remaining slots)
  const int tstride = nquad * kCPQ * 96;  // limbs of one token
  uint8_t* xq = lds + 512;
  i32x4* meta = reinterpret_cast<i32x4*>(xq + MT * tstride);
  uint16_t* yl = reinterpret_cast<uint16_t*>(meta + MT * nquad * 4);
  float* part = reinterpret_cast<float*>(yl + ((MT * nb * 4 + 3) & ~3));
  int* tickets = reinterpret_cast<int*>(part + (SPLIT > 1 ? nb * P * MT * 4 : 0));

  if (SPLIT > 1)
    for (int i = tid; i < nb; i += 64 * nwv) tickets[i] = 0;
  if (tid < 128) reinterpret_cast<uint32_t*>(lds)[tid] = 0u;

  // ---- activations, step 1: this lane's bf16 inputs, requested and waited for before any weight request (behind
  // the weight requests of the whole GPU, x would arrive microseconds late)
  const int gpt = nquad * 4;  // groups per token
  const int sub = lane % LPU, units = gpt * MT, ustride = nwv * UPW;
  const int u0 = wave * UPW + lane / LPU;
  const int npass = (units + ustride - 1) / ustride;
  uint4 xv[XB];
  auto xload = [&](int pass0) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      // lanes past the end load x[0] (zero-selected); passes past npass load nothing (a wave-uniform branch)
      const int u = u0 + (pass0 + b) * ustride, t = MT == 1 ? 0 : u / gpt, kk = (u - t * gpt) * kG + 8 * sub;
      const bool ok = u < units && t < mm && kk < k;
      xv[b] = make_uint4(0u, 0u, 0u, 0u);
      if (pass0 + b < npass) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.x + (ok ? (size_t)t * k + kk : 0));
        xv[b] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  AK_M1_STAMP(0);
  xload(0);
#pragma unroll
  for (int b = 0; b < XB; ++b) asm volatile("" ::"v"(xv[b].x), "v"(xv[b].y), "v"(xv[b].z), "v"(xv[b].w));
  AK_M1_STAMP(1);

  // ---- this wave's tasks: stripe set j, quads [qa, qb), block groups b0w, b0w + bstep, ... < ng (a group is RB
  // consecutive blocks: an item loads the same quad of each, and they share its activation operand)
  const int ng = (nb + RB - 1) / RB;
  const int j = wave % SPLIT, bstep = nwv / SPLIT, b0w = wave / SPLIT;
  const int pa = j * P / SPLIT, pb = (j + 1) * P / SPLIT;
  const int qa = stripe_begin(pa, nquad, P), qb = stripe_begin(pb, nquad, P);
  const int ntw = b0w < ng ? (ng - b0w + bstep - 1) / bstep : 0;
  const int nitems = ntw * (qb - qa);
  // bit q - qa set when quad q is the last of its stripe (quads < qa + 128)
  unsigned long long ends0 = 0, ends1 = 0;
  for (int p = pa; p < pb; ++p) {
    const int r = stripe_begin(p + 1, nquad, P) - 1 - qa;
    if (r < 64) ends0 |= 1ull << r;
    else ends1 |= 1ull << (r - 64);
  }

  // ---- weight addressing: per lane fixed, per item scalar.  Rows past the segment's end (padding of the last block)
  // read other rows or, past the buffer, zeros; their results are not written.
  const int tiles = kpad(k) >> 10;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(AK_PICK(sg, sgs.wt)), (short)0, tiles * n * REC, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(AK_PICK(sg, sgs.st)), (short)0, tiles * n * 16, kRsrcWord3);
  const int ch = 4 * vv + h;  // this lane's chunk within the 16 of a quad
  const int vo_w = rr * REC + ch * CHB, vo_h = rr * REC + 256 + ch * 4, vo_s = rr * 16 + (vv & 2) * 2;
  const int tile_w = n * REC, tile_s = n * 16;
  auto fetch1 = [&](int blk, int qd, Raw<BITS>& dst, uint32_t& sdst) {
    const int row0 = (b_lo + blk) * 4;
    const int so = row0 * REC + (qd >> 1) * tile_w, odd = qd & 1;
    if constexpr (BITS == 4) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, so + odd * 256, kNt);
      dst.w = make_uint4(v[0], v[1], v[2], v[3]);
    } else {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, vo_w, so + odd * 128, kNt);
      dst.lo = make_uint2(v[0], v[1]);
      if constexpr (BITS == 3) dst.hi = __builtin_amdgcn_raw_buffer_load_b32(rw, vo_h, so + odd * 64, kNt);
    }
    // the aligned dword holding the scale (the item selects its half): a 16-bit value would be widened or packed at
    // the loop latch, which waits for the load
    sdst = __builtin_amdgcn_raw_buffer_load_b32(rs, vo_s, row0 * 16 + (qd >> 1) * tile_s + odd * 8, 0);
  };
  auto fetch = [&](int grp, int qd, Raw<BITS> (&dst)[RB], uint32_t (&sdst)[RB]) {
#pragma unroll
    for (int r = 0; r < RB; ++r) fetch1(grp * RB + r, qd, dst[r], sdst[r]);
  };

  Raw<BITS> buf[DEPTH][RB];
  uint32_t sbuf[DEPTH][RB];

  // fetch cursor (an item past the end reloads quad qa of block 0: cache-resident, never used, and the load sequence
  // stays branch-free so the compiler's load counters stay exact)
  int fb = b0w, fq = qa;
  auto fetch_next = [&](Raw<BITS> (&dst)[RB], uint32_t (&sdst)[RB]) {
    const bool in = fb < ng;
    fetch(in ? fb : 0, in ? fq : qa, dst, sdst);
    const bool wrap = fq + 1 == qb;
    fq = wrap ? qa : fq + 1;
    fb = wrap ? fb + bstep : fb;
  };

  // ---- the first DEPTH items are requested, then step 2 of the activations: per group the limbs (to LDS), and in
  // meta the bias sums -OFF * sum(d_j) of the three limbs with the activation scale 2^(E - 148) as float bits
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) fetch_next(buf[d], sbuf[d]);

  auto convert = [&](int p0) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      if (p0 + b >= npass) break;
      const int u = u0 + (p0 + b) * ustride;
      uint32_t t0[8], t1[8], t2[8];
      const int e = group_limbs<LPU>(xv[b], t0, t1, t2);
      const int b0 = dpp_group_reduce<LPU, false>(limb_sum8(t0, 0));
      const int b1 = dpp_group_reduce<LPU, false>(limb_sum8(t1, 1));
      const int b2 = dpp_group_reduce<LPU, false>(limb_sum8(t2, 2));
      if (u < units) {
        const int t = MT == 1 ? 0 : u / gpt, ut = u - t * gpt;
        const int qd = ut >> 2, gq = ut & 3, eg0 = 8 * sub, cqd = gq * 4 + (eg0 >> 5);
        store_limbs<BITS>(xq + t * tstride + qd * kCPQ * 96 + cqd * 48, kCPQ * 48, eg0 & 31, t0, t1, t2);
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
    xload(p0);
    convert(p0);
  }
  __syncthreads();
  AK_M1_STAMP(2);

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

  // compute cursor: block, quad, stripe
  int cb = b0w, cq = qa, cp = pa;
  float acc[RB][MT], yrun[RB][MT];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[r][t] = 0.f, yrun[r][t] = 0.f;
  // one item without branches: an[][] = the accumulators before a stripe end reset them (used only at a stripe end)
  auto core = [&](const Raw<BITS> (&bf)[RB], const uint32_t (&sraw)[RB], float (&an)[RB][MT], bool& end, int& eg,
                  int& ep) {
    const int r0 = cq - qa;
    end = ((r0 < 64 ? ends0 >> r0 : ends1 >> (r0 - 64)) & 1ull) != 0;
    i32x4 b0[RB], b1[RB];
    float sc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      sc[r] = __uint_as_float(__builtin_amdgcn_perm(sraw[r], sraw[r], ssel));
      make_b<BITS>(bf[r], b0[r], b1[r]);
    }
    // token by token: the activation operand and meta of one token are live at a time
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const i32x4 mt = meta[(t * nquad + cq) * 4 + h];
      const uint8_t* src = lds + a_base + t * a_tmul + cq * a_qmul;
      const i32x4 a0 = *reinterpret_cast<const i32x4*>(src);
      const i32x4 a1 = *reinterpret_cast<const i32x4*>(src + (a_on ? kCPQ * 48 : 0));
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        i32x4 d = mt;
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0[r], d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1[r], d, 0, 0, 0);
        an[r][t] = fmaf(group_sum_f32(d), sc[r] * __int_as_float(mt[3]), acc[r][t]);
        acc[r][t] = end ? 0.f : an[r][t];
      }
    }
    eg = cb;
    ep = cp;
    cp = end ? cp + 1 : cp;
    const bool wrap = cq + 1 == qb;
    cq = wrap ? qa : cq + 1;
    cb = wrap ? cb + bstep : cb;
    cp = wrap ? pa : cp;
  };
  // a stripe ended with accumulators v[][]: its partial per row (lanes 0..3: ((slot 0 + slot 1) + slot 2) + slot 3,
  // slot v of row r in lane 17v + 4r), then the blocks' outputs when the task ends
  auto stripe_end = [&](const float (&v)[RB][MT], int eg, int ep) {
    float pp[RB][MT];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int vi = __float_as_int(v[r][t]);
        const float v0 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl0, vi)),
                    v1 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl1, vi)),
                    v2 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl2, vi)),
                    v3 = __int_as_float(__builtin_amdgcn_ds_bpermute(sl3, vi));
        pp[r][t] = ((v0 + v1) + v2) + v3;
      }
    if constexpr (SPLIT == 1) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          yrun[r][t] = ep == 0 ? pp[r][t] : yrun[r][t] + pp[r][t];
          if (ep == P - 1 && eg * RB + r < nb) write_y(eg * RB + r, t, yrun[r][t]);
        }
    } else {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          if (lane < 4 && eg * RB + r < nb) part[(((eg * RB + r) * P + ep) * MT + t) * 4 + lane] = pp[r][t];
      if (ep + 1 < pb) return;  // more stripes in this task
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  // LDS only: no wait for loads in flight
      int last = 0;
      if (lane == 0) last = atomicAdd(&tickets[eg], 1) == SPLIT - 1;
      last = __shfl(last, 0);
      if (last) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          if (eg * RB + r >= nb) continue;
          const float* slot = part + (eg * RB + r) * P * MT * 4;
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            float y = slot[t * 4 + (lane & 3)];
            for (int q = 1; q < P; ++q) y += slot[(q * MT + t) * 4 + (lane & 3)];
            write_y(eg * RB + r, t, y);
          }
        }
      }
    }
  };

  const int nfull = nitems / DEPTH * DEPTH;
  for (int i0 = 0; i0 < nfull; i0 += DEPTH) {
    float sv[DEPTH][RB][MT];
    bool end[DEPTH];
    int eg[DEPTH], ep[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      core(buf[d], sbuf[d], sv[d], end[d], eg[d], ep[d]);
      fetch_next(buf[d], sbuf[d]);
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (end[d]) stripe_end(sv[d], eg[d], ep[d]);
  }
  // the last, partial group (its later fetches load the cache-resident dummy item)
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    if (nfull + d < nitems) {
      float v[RB][MT];
      bool e;
      int g, p;
      core(buf[d], sbuf[d], v, e, g, p);
      if (e) stripe_end(v, g, p);
    }
  }
  AK_M1_STAMP(3);
  __syncthreads();
  for (int i = tid; i < MT * nb * 4; i += 64 * nwv) {
    const int t = MT == 1 ? 0 : i / (nb * 4), row = b_lo * 4 + i - t * nb * 4;
    if (t < mm && row < n) yseg[(size_t)t * ldy + row] = yl[i];
  }
}

size_t m1d_x_bytes(int nquad, int mt) { return 512 + (size_t)mt * nquad * (kCPQ * 96 + 4 * 16); }
size_t m1d_block_bytes(int P, int split, int mt) {  // per 4-row block: outputs, partials, ticket
  return (size_t)mt * 8 + (split > 1 ? (size_t)P * 16 * mt + 4 : 0);
}

template <int BITS, int SPLIT, int RB, int MT>
void launch_split(const I8Args& a, int grid, int nwv, size_t smem, hipStream_t s) {
  constexpr int DEPTH = RB * MT <= 2 ? 4 / RB : 2;  // items in flight per wave
  hipLaunchKernelGGL((i8_m1d_kernel<BITS, SPLIT, DEPTH, RB, MT>), dim3(grid), dim3(64 * nwv), smem, s, a);
}

template <int BITS, int MT>
int launch_m1d(I8Args a, hipStream_t s) {
  const Segs& g = a.segs;
  const size_t x_bytes = m1d_x_bytes(a.nquad, MT);
  const int tiles = kpad(a.k) >> 10;
  for (int i = 0; i < g.nseg; ++i)  // buffer offsets are 32-bit
    if ((long long)tiles * g.n[i] * 128 * BITS >= (1ll << 31)) return AK_INVALID;
  if (x_bytes > 150 * 1024) return AK_INVALID;
  // workgroups per segment: about the same number of blocks each, at most one workgroup per CU
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
  // waves per workgroup, waves per block and blocks per item: fewest item rounds for the busiest wave, a task's
  // overhead counted as about one item and a two-block item as 1.7 items; ties go to more waves (latency hiding),
  // fewer waves per block (less exchange) and single blocks (finer balance)
  int best_split = 1, best_nwv = 16, best_rb = 1;
  double best = 1e30;
  for (int rb : {1, 2})
    for (int nwv : {16, 8}) {
      if (MT > 1 && rb > 1) continue;
      for (int split : {1, 2, 4, 8}) {
        if (split > a.P) break;
        if (x_bytes + (size_t)nbmax * m1d_block_bytes(a.P, split, MT) + 16 > 160 * 1024) continue;
        int lmax = 0;
        for (int j = 0; j < split; ++j) {
          const int l =
              stripe_begin((j + 1) * a.P / split, a.nquad, a.P) - stripe_begin(j * a.P / split, a.nquad, a.P);
          lmax = l > lmax ? l : lmax;
        }
        const int bstep = nwv / split, ngmax = (nbmax + rb - 1) / rb;
        const double cost = (double)((ngmax + bstep - 1) / bstep) * (lmax * (rb == 1 ? 1.0 : 1.7) + 1.0);
        if (cost < best - 1e-9) best = cost, best_split = split, best_nwv = nwv, best_rb = rb;
      }
    }
  if (best > 1e29) return AK_INVALID;
  const size_t smem = x_bytes + (size_t)nbmax * m1d_block_bytes(a.P, best_split, MT) + 16;
  if constexpr (MT == 1) {
    switch (best_split * 10 + best_rb) {
      case 11: launch_split<BITS, 1, 1, 1>(a, grid, best_nwv, smem, s); break;
      case 21: launch_split<BITS, 2, 1, 1>(a, grid, best_nwv, smem, s); break;
      case 41: launch_split<BITS, 4, 1, 1>(a, grid, best_nwv, smem, s); break;
      case 81: launch_split<BITS, 8, 1, 1>(a, grid, best_nwv, smem, s); break;
      case 12: launch_split<BITS, 1, 2, 1>(a, grid, best_nwv, smem, s); break;
      case 22: launch_split<BITS, 2, 2, 1>(a, grid, best_nwv, smem, s); break;
      case 42: launch_split<BITS, 4, 2, 1>(a, grid, best_nwv, smem, s); break;
      default: launch_split<BITS, 8, 2, 1>(a, grid, best_nwv, smem, s); break;
    }
  } else {
    switch (best_split) {
      case 1: launch_split<BITS, 1, 1, MT>(a, grid, best_nwv, smem, s); break;
      case 2: launch_split<BITS, 2, 1, MT>(a, grid, best_nwv, smem, s); break;
      case 4: launch_split<BITS, 4, 1, MT>(a, grid, best_nwv, smem, s); break;
      default: launch_split<BITS, 8, 1, MT>(a, grid, best_nwv, smem, s); break;
    }
  }
  return (int)hipGetLastError();
}

}  // namespace

// up to 8 tokens (padded to 1, 2, 4 or 8 in the kernel); each segment's rows are processed in 4-row blocks (the last
// one padded).  Returns AK_INVALID if the shape does not suit the kernel (group 64, the tokens' activations beyond the
// LDS, a segment beyond 2 GB): the caller falls back to the any-m kernel.
int i8_gemv_m1(int bits, const void* x, int m, const Segs& g, int k, int group, hipStream_t s) {
  if (group != kG || m < 1 || m > 8) return AK_INVALID;
  I8Args a;
  a.segs = g;
  a.x = static_cast<const uint16_t*>(x);
  a.m = m;
  a.k = k;
  a.nquad = kpad(k) / kG / 4;
  a.P = a.nquad < 8 ? a.nquad : 8;
  a.nb = 0;
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

}  // namespace agq
