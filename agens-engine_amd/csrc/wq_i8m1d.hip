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
// Work decomposition: one persistent workgroup per CU owns a contiguous range of 4-row blocks.  Its tasks are
// (block, stripe set j < SPLIT) pairs, dealt round-robin to the waves; a task runs the stripes j, j + SPLIT, ... of
// its block one after the other, each over the quads p, p + P, ... (the fp32 order of the numerics).  With SPLIT = 1 a
// wave owns whole blocks and adds the stripe partials itself; otherwise the partials meet in LDS and the last task of
// a block to finish (LDS ticket) adds them in stripe order.  Every wave streams its items (one quad of one block: one
// buffer load per lane, two for W3, plus one for the scales) through DEPTH register buffers; each item's offsets are
// wave-uniform (scalar registers) on top of per-lane offsets fixed for the task.
#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_i8_common.h"

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

// a wave's position in its task list
struct Cursor {
  int t;   // task, local to the workgroup
  int b;   // block, local to the workgroup
  int p;   // stripe
  int qd;  // quad
};

template <int BITS, int SPLIT, int DEPTH>
__global__ void __launch_bounds__(1024, 1) i8_m1d_kernel(const I8Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int LPU = kG / 8, UPW = 64 / LPU, XB = 4;
  const int P = a.P, nquad = a.nquad, k = a.k;
  const int nwv = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int rr = c >> 2, vv = c & 3;  // B role: row of the block, group of the quad
  const Segs& sgs = a.segs;
  const int n_b4 = sgs.end[sgs.nseg - 1] >> 2;
  const int b_lo = (int)((long long)blockIdx.x * n_b4 / gridDim.x);
  const int nb = (int)((long long)(blockIdx.x + 1) * n_b4 / gridDim.x) - b_lo;
  const int ntask = nb * SPLIT;

  // LDS: zeros [512 B] | limbs [nquad][16][2][3][16 B] | meta [nquad][4] int4 | outputs [nb][4] bf16 |
  //      partials [nb][P][4] | tickets [nb]
  uint8_t* xq = lds + 512;
  i32x4* meta = reinterpret_cast<i32x4*>(xq + nquad * kCPQ * 96);
  uint16_t* yl = reinterpret_cast<uint16_t*>(meta + nquad * 4);
  float* part = reinterpret_cast<float*>(yl + ((nb * 4 + 3) & ~3));
  int* tickets = reinterpret_cast<int*>(part + (SPLIT > 1 ? nb * P * 4 : 0));

  if (SPLIT > 1)
    for (int i = tid; i < nb; i += 64 * nwv) tickets[i] = 0;
  if (tid < 128) reinterpret_cast<uint32_t*>(lds)[tid] = 0u;

  // ---- activations, step 1: this lane's bf16 inputs, requested and waited for before any weight request (behind
  // the weight requests of the whole GPU, x would arrive microseconds late)
  const int sub = lane % LPU, units = nquad * 4, ustride = nwv * UPW;
  const int u0 = wave * UPW + lane / LPU;
  const int npass = (units + ustride - 1) / ustride;
  uint4 xv[XB];
  auto xload = [&](int pass0) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      const int u = u0 + (pass0 + b) * ustride, kk = u * kG + 8 * sub;
      const bool ok = u < units && kk < k;
      xv[b] = make_uint4(0u, 0u, 0u, 0u);
      if (pass0 + b < npass) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.x + (ok ? kk : 0));
        xv[b] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  xload(0);
#pragma unroll
  for (int b = 0; b < XB; ++b) asm volatile("" ::"v"(xv[b].x), "v"(xv[b].y), "v"(xv[b].z), "v"(xv[b].w));

  // ---- task walk.  Task t: block t / SPLIT, stripe set t % SPLIT; a wave takes tasks wave, wave + nwv, ...
  auto start = [&](Cursor& x, int t) {
    x.t = t;
    x.b = t / SPLIT;
    x.p = t % SPLIT;
    x.qd = x.p;
  };
  auto advance = [&](Cursor& x) {
    x.qd += P;
    if (x.qd >= nquad) {
      x.p += SPLIT;
      if (x.p >= P) {
        start(x, x.t + nwv);
      } else {
        x.qd = x.p;
      }
    }
  };
  // items of this wave
  int nitems = 0;
  for (int t = wave; t < ntask; t += nwv)
    for (int p = t % SPLIT; p < P; p += SPLIT) nitems += (nquad - p + P - 1) / P;

  // per-task buffer addressing of the fetch cursor: resources of the block's segment and this lane's offsets
  struct Addr {
    __amdgpu_buffer_rsrc_t w, s;
    int vo_w, vo_h, vo_s;  // per lane: weights (W3: two-bit planes), W3 third-bit plane, scale dword
    int tile_w, tile_s;    // bytes between 1024-input tiles of the segment (n records / n scale rows)
  };
  const int tiles = kpad(k) >> 10;
  auto address = [&](int bl, Addr& ad) {
    const int g0 = (b_lo + (bl < nb ? bl : 0)) * 4;
    const int sg = seg_of(sgs, g0);
    const int n = AK_PICK(sg, sgs.n);
    int orow = g0 - (sg ? AK_PICK(sg - 1, sgs.end) : 0) + rr;
    if (orow >= n) orow = 0;  // padding rows read row 0 (results unused)
    ad.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(AK_PICK(sg, sgs.wt)), (short)0,
                                             tiles * n * Rec<BITS>::bytes, kRsrcWord3);
    ad.s = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(AK_PICK(sg, sgs.st)), (short)0, tiles * n * 16,
                                             kRsrcWord3);
    const int ch = 4 * vv + h;  // this lane's chunk within the 16 of a quad
    ad.vo_w = orow * Rec<BITS>::bytes + ch * Rec<BITS>::chunk;
    ad.vo_h = orow * Rec<BITS>::bytes + 256 + ch * 4;
    ad.vo_s = orow * 16 + (vv & 2) * 2;
    ad.tile_w = n * Rec<BITS>::bytes;
    ad.tile_s = n * 16;
  };
  // one item: its weights and the dword holding its scale (an item past the end reloads quad 0: cache-resident, never
  // used, and it keeps the load sequence branch-free so the compiler's load counters stay exact)
  auto fetch = [&](const Cursor& x, const Addr& ad, Raw<BITS>& dst, uint32_t& sdst) {
    const int qd = x.t < ntask ? x.qd : 0;
    const int so = (qd >> 1) * ad.tile_w, odd = qd & 1;
    if constexpr (BITS == 4) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(ad.w, ad.vo_w, so + odd * 256, kNt);
      dst.w = make_uint4(v[0], v[1], v[2], v[3]);
    } else {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(ad.w, ad.vo_w, so + odd * 128, kNt);
      dst.lo = make_uint2(v[0], v[1]);
      if constexpr (BITS == 3) dst.hi = __builtin_amdgcn_raw_buffer_load_b32(ad.w, ad.vo_h, so + odd * 64, kNt);
    }
    sdst = __builtin_amdgcn_raw_buffer_load_b32(ad.s, ad.vo_s, (qd >> 1) * ad.tile_s + odd * 8, 0);
  };

  Raw<BITS> buf[DEPTH];
  uint32_t sbuf[DEPTH];

  // ---- the first DEPTH items are requested, then step 2 of the activations: per group the limbs (to LDS), and in
  // meta the bias sums -OFF * sum(d_j) of the three limbs with the activation scale 2^(E - 148) as float bits
  Cursor fc;
  start(fc, wave);
  Addr fa;
  address(fc.b, fa);
  auto fetch_next = [&](Raw<BITS>& dst, uint32_t& sdst) {
    fetch(fc, fa, dst, sdst);
    const int t0 = fc.t;
    advance(fc);
    if (fc.t != t0) address(fc.b, fa);
  };
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
        const int qd = u >> 2, gq = u & 3, eg0 = 8 * sub, cq = gq * 4 + (eg0 >> 5);
        store_limbs<BITS>(xq + (qd * kCPQ + cq) * 96, 48, eg0 & 31, t0, t1, t2);
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

  // A role: group c >> 2, limb c & 3 (limb 3 reads the zero region), chunk 4 * (c >> 2) + h of the quad
  const bool a_on = (c & 3) < 3;
  const int a_base = a_on ? 512 + (4 * (c >> 2) + h) * 96 + 16 * (c & 3) : 0;
  const int a_qmul = a_on ? kCPQ * 96 : 0;

  // outputs are staged in LDS and written after the loop: a global store among the streaming loads would make the
  // compiler drain every load in flight
  auto write_y = [&](int bl, float y) {  // lanes 0..3: row `lane` of local block bl
    if (lane < 4) yl[bl * 4 + lane] = f2bf(y);
  };

  float acc = 0.f, yrun = 0.f;
  auto item = [&](const Cursor& x, const Raw<BITS>& bf, uint32_t sraw) {
    const int qd = x.qd, p = x.p;
    if (qd == p) acc = 0.f;  // first quad of this stripe
    i32x4 d = meta[qd * 4 + h];
    const float sE = __uint_as_float(vv & 1 ? sraw & 0xFFFF0000u : sraw << 16) * __int_as_float(d[3]);
    i32x4 b0, b1;
    make_b<BITS>(bf, b0, b1);
    const uint8_t* src = lds + a_base + qd * a_qmul;
    const i32x4 a0 = *reinterpret_cast<const i32x4*>(src);
    const i32x4 a1 = *reinterpret_cast<const i32x4*>(src + 48);
    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
    acc = fmaf(group_sum_f32(d), sE, acc);
    if (qd + P < nquad) return;  // more quads in this stripe
    // stripe partial of row r = lane (lanes 0..3): ((slot 0 + slot 1) + slot 2) + slot 3, slot v in lane 17 v + 4 r
    const int r4 = 4 * (lane & 3);
    const float v0 = __shfl(acc, r4), v1 = __shfl(acc, 17 + r4), v2 = __shfl(acc, 34 + r4), v3 = __shfl(acc, 51 + r4);
    const float pp = ((v0 + v1) + v2) + v3;
    if constexpr (SPLIT == 1) {
      yrun = p == 0 ? pp : yrun + pp;
      if (p == P - 1) write_y(x.b, yrun);
    } else {
      float* slot = part + x.b * P * 4;
      if (lane < 4) slot[p * 4 + lane] = pp;
      if (p + SPLIT < P) return;  // more stripes in this task
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  // LDS only: no wait for loads in flight
      int last = 0;
      if (lane == 0) last = atomicAdd(&tickets[x.b], 1) == SPLIT - 1;
      last = __shfl(last, 0);
      if (last) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        float y = slot[lane & 3];
        for (int q = 1; q < P; ++q) y += slot[q * 4 + (lane & 3)];
        write_y(x.b, y);
      }
    }
  };

  // full rounds of DEPTH: the compute of an item past the end is skipped (a wave-uniform branch that leaves the
  // buffers alone), its fetch is not, so the buffer registers stay fixed and the load counters exact
  Cursor cc;
  start(cc, wave);
  for (int i0 = 0; i0 < nitems; i0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      if (i0 + d < nitems) item(cc, buf[d], sbuf[d]);
      fetch_next(buf[d], sbuf[d]);
      advance(cc);
    }
  }
  __syncthreads();
  for (int i = tid; i < nb * 4; i += 64 * nwv) {
    const int g = b_lo * 4 + i;
    const int sg = seg_of(sgs, g);
    const int orow = g - (sg ? AK_PICK(sg - 1, sgs.end) : 0);
    if (orow < AK_PICK(sg, sgs.n)) AK_PICK(sg, sgs.y)[orow] = yl[i];
  }
}

size_t m1d_x_bytes(int nquad) { return 512 + (size_t)nquad * (kCPQ * 96 + 4 * 16); }
size_t m1d_block_bytes(int P, int split) { return 8 + (split > 1 ? (size_t)P * 16 + 4 : 0); }  // per 4-row block

template <int BITS, int SPLIT>
void launch_split(const I8Args& a, int grid, int nwv, size_t smem, hipStream_t s) {
  constexpr int DEPTH = 8;  // items in flight per wave
  hipLaunchKernelGGL((i8_m1d_kernel<BITS, SPLIT, DEPTH>), dim3(grid), dim3(64 * nwv), smem, s, a);
}

template <int BITS>
int launch_m1d(const I8Args& a, hipStream_t s) {
  const int n_b4 = a.segs.end[a.segs.nseg - 1] / 4;
  const size_t x_bytes = m1d_x_bytes(a.nquad);
  const int tiles = kpad(a.k) >> 10;
  for (int i = 0; i < a.segs.nseg; ++i)  // buffer offsets are 32-bit
    if ((long long)tiles * a.segs.n[i] * 128 * BITS >= (1ll << 31)) return AK_INVALID;
  if (x_bytes > 150 * 1024) return AK_INVALID;
  const int grid = n_b4 < num_cus() ? n_b4 : num_cus();
  const int nbmax = (n_b4 + grid - 1) / grid;
  // waves per workgroup and waves per block: fewest item rounds of the busiest wave, counting a task's overhead as
  // about one item; ties go to more waves (latency hiding) and to fewer waves per block (less exchange)
  int best_split = 1, best_nwv = 16;
  double best = 1e30;
  for (int nwv : {16, 12, 8})
    for (int split : {1, 2, 4, 8}) {
      if (split > a.P) break;
      if (x_bytes + (size_t)nbmax * m1d_block_bytes(a.P, split) + 16 > 160 * 1024) continue;
      const int tasks = nbmax * split;
      const int per_wave = (tasks + nwv - 1) / nwv;
      const int items = (a.P + split - 1) / split * ((a.nquad + a.P - 1) / a.P);
      const double cost = per_wave * (items + 1.0);
      if (cost < best - 1e-9) best = cost, best_split = split, best_nwv = nwv;
    }
  if (best > 1e29) return AK_INVALID;
  const size_t smem = x_bytes + (size_t)nbmax * m1d_block_bytes(a.P, best_split) + 16;
  switch (best_split) {
    case 1: launch_split<BITS, 1>(a, grid, best_nwv, smem, s); break;
    case 2: launch_split<BITS, 2>(a, grid, best_nwv, smem, s); break;
    case 4: launch_split<BITS, 4>(a, grid, best_nwv, smem, s); break;
    default: launch_split<BITS, 8>(a, grid, best_nwv, smem, s); break;
  }
  return (int)hipGetLastError();
}

}  // namespace

// one token, group 128; the segments' row ranges are re-padded to 4 rows.  Returns AK_INVALID if the shape does not
// suit the kernel (activations beyond the LDS, a segment beyond 2 GB): the caller falls back.
int i8_gemv_m1d(int bits, const void* x, const Segs& g0, int k, hipStream_t s) {
  Segs g = g0;
  for (int i = 0, e = 0; i < g.nseg; ++i) {
    e += (g.n[i] + 3) / 4 * 4;
    g.end[i] = e;
  }
  I8Args a;
  a.segs = g;
  a.x = static_cast<const uint16_t*>(x);
  a.m = 1;
  a.k = k;
  a.nquad = kpad(k) / kG / 4;
  a.P = a.nquad < 8 ? a.nquad : 8;
  a.nb = 0;
  a.iters_max = 1;
  switch (bits) {
    case 4: return launch_m1d<4>(a, s);
    case 3: return launch_m1d<3>(a, s);
    case 2: return launch_m1d<2>(a, s);
    default: return AK_INVALID;
  }
}

}  // namespace agq
