// The default-numerics GEMV for one token (decode, M = 1) on gfx950: the same exact integer group sums and the same
// fp32 accumulation order as wq_i8.hip (so its rows are bit-identical to any-m launches), with an MFMA layout made for
// a single activation vector:
//
//   "groups in rows": A row 4u + j = limb j of GROUP u of a quad (not of token u), and lane group h of the B operand
//   feeds group h (step s of a quad takes chunk s of each of the four groups).  Lanes whose A row belongs to another
//   group hold 0, so one MFMA chain over a quad yields the limb sums of all four groups at once, and every lane's
//   combine (group sum -> fp32, times scale) is useful work: lane (r, h) owns output row r, group slot h.
//
// Work decomposition: persistent workgroups of NWV waves.  The whole activation vector is converted once per
// workgroup into LDS (limbs, bias sums, activation scales), then every wave streams "items" (one quad of one 16-row
// block) through two register buffers, two items ahead, with no further barrier.  SWD waves share a row block by
// splitting its stripes (for small n, to use the whole GPU); their stripe partials meet in LDS and the last wave to
// arrive (LDS atomic ticket) adds them in stripe order.  With SWD = 1 a wave owns whole row blocks.
#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_i8_common.h"

// phase timestamps for profiling builds (a build that defines it records them; product builds compile nothing)
#ifndef AK_M1_STAMP
#define AK_M1_STAMP(i)
#define AK_M1_STAMP_AFTER(i, v)
#endif

namespace agq {

int num_cus();

namespace {

struct ItemPos {
  int it, ls, qd;
  int valid;  // an int, not a bool: a padded struct is copied through scratch memory
};

template <int BITS, int G, int SWD, int NWV, int WPE>
__global__ void __launch_bounds__(64 * NWV, WPE) i8_m1_kernel(const I8Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int CPG = G / 32, CPQ = 4 * CPG, SPT = 1024 / G, LPU = G / 8;
  constexpr int RWV = NWV / SWD;             // row blocks per workgroup iteration
  constexpr int NPW = (8 + SWD - 1) / SWD;   // most stripes of one wave
  const int P = a.P, nquad = a.nquad, k = a.k;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps the item bookkeeping scalar
  const int sw = wave % SWD, rw = wave / SWD;
  const int r = lane & 15, h = lane >> 4;
  const Segs& sgs = a.segs;
  const int rows_pad = sgs.end[sgs.nseg - 1];
  const int n_rb = rows_pad >> 4;

  // LDS: zeros [512 B] | limbs [nquad][CPQ][2][3][16 B] | meta [nquad][4] int4 | partials | tickets
  uint8_t* xq = lds + 512;
  i32x4* meta = reinterpret_cast<i32x4*>(xq + nquad * CPQ * 96);
  float* part = reinterpret_cast<float*>(meta + nquad * 4);  // [iters_max][RWV][8][16]
  int* tickets = reinterpret_cast<int*>(part + (SWD > 1 ? a.iters_max * RWV * 8 * 16 : 0));

  auto row_info = [&](int rb, const void*& wt, const uint16_t*& st, int& n, int& orow, bool& ok) {
    const int g0 = rb * 16;
    const int sg = seg_of(sgs, g0);
    n = sgs.n[sg];
    orow = g0 - (sg ? sgs.end[sg - 1] : 0) + r;
    ok = orow < n;
    if (!ok) orow = 0;  // padding rows load row 0 of the segment (results unused)
    wt = sgs.wt[sg];
    st = sgs.st[sg];
  };
  auto first = [&]() {
    ItemPos x;
    x.it = blockIdx.x, x.ls = 0, x.qd = sw;
    x.valid = x.it * RWV + rw < n_rb;
    return x;
  };
  auto advance = [&](ItemPos& x) {
    x.qd += P;
    if (x.qd >= nquad) {
      ++x.ls;
      int p = x.ls * SWD + sw;
      if (x.ls >= NPW || p >= P) {
        x.it += gridDim.x, x.ls = 0, p = sw;
        x.valid = x.it * RWV + rw < n_rb;
      }
      x.qd = p;
    }
  };
  auto fetch = [&](const ItemPos& x, Raw<BITS>(&dst)[CPG], uint32_t& sdst) {
    // branch-free: an invalid item (past the end) loads row block 0 (L2-resident, never used), so the compiler keeps
    // exact load counters across the fetches instead of draining every outstanding load at a control-flow merge
    const void* wt;
    const uint16_t* st;
    int n, orow;
    bool ok;
    row_info(x.valid ? x.it * RWV + rw : 0, wt, st, n, orow, ok);
    const int cg0 = x.qd * CPQ + h * CPG;  // this lane group's group: chunks cg0 .. cg0 + CPG - 1 (one tile)
    const size_t rec = (size_t)(cg0 >> 5) * n + orow;
#pragma unroll
    for (int s = 0; s < CPG; ++s) dst[s] = load_raw<BITS>(wt, rec, (cg0 & 31) + s);
    const int g = x.qd * 4 + h;
    sdst = st[((size_t)(g / SPT) * n + orow) * SPT + (g % SPT)];
  };

  if (SWD > 1)
    for (int i = tid; i < a.iters_max * RWV; i += 64 * NWV) tickets[i] = 0;
  if (tid < 128) reinterpret_cast<uint32_t*>(lds)[tid] = 0u;

  // ---- activations, step 1: every lane's bf16 inputs are requested first (x is small and mostly L2-resident), then
  // the first two weight items, so that waiting for x does not wait for the weights.
  constexpr int UPW = 64 / LPU, XB = 8;  // groups per wave and pass, passes per load batch
  const int sub = lane % LPU, units = nquad * 4, ustride = NWV * UPW;
  const int u0 = wave * UPW + lane / LPU;
  const int npass = (units + ustride - 1) / ustride;
  uint4 xv[XB];
  auto xload = [&](int pass0) {
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      // unconditional loads (clamped address, zero-selected) keep the load sequence branch-free
      // lanes past the end load x[0] (zero-selected); passes past npass load nothing (a wave-uniform branch)
      const int u = u0 + (pass0 + b) * ustride, kk = u * G + 8 * sub;
      const bool ok = u < units && kk < k;
      xv[b] = make_uint4(0u, 0u, 0u, 0u);
      if (pass0 + b < npass) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.x + (ok ? kk : 0));
        xv[b] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  AK_M1_STAMP(0);
  xload(0);
  AK_M1_STAMP_AFTER(1, lane);
  // wait for x before requesting weights: behind the weight requests of the whole GPU, x (one cache line per XCD to
  // miss) would arrive microseconds late
#pragma unroll
  for (int b = 0; b < XB; ++b) asm volatile("" ::"v"(xv[b].x), "v"(xv[b].y), "v"(xv[b].z), "v"(xv[b].w));

  ItemPos pa = first(), pb = pa;
  advance(pb);
  pb.valid = pb.valid && pa.valid;
  Raw<BITS> buf0[CPG], buf1[CPG];
  uint32_t s0 = 0, s1 = 0;
  fetch(pa, buf0, s0);
  fetch(pb, buf1, s1);

  // ---- activations, step 2: per group the limbs (to LDS), and in meta the bias sums -OFF * sum(d_j) of the three
  // limbs with the activation scale 2^(E - 148) as float bits
  auto convert = [&](int p0) {
    AK_M1_STAMP_AFTER(2, xv[0].x);
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
        const int qd = u >> 2, gq = u & 3, eg0 = 8 * sub, cq = gq * CPG + (eg0 >> 5);
        store_limbs<BITS>(xq + (qd * CPQ + cq) * 96, 48, eg0 & 31, t0, t1, t2);
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
  const int limb_a = r & 3, ua = r >> 2;
  const bool a_on = limb_a < 3 && ua == h;  // A row 4u + j is fed only by lane group u
  // branch-free A reads: inactive lanes read the zeroed region at the start of the LDS (quad offset forced to 0)
  const int a_base = a_on ? 512 + (h * CPG * 96 + 16 * limb_a) : 0;
  const int a_qmul = a_on ? CPQ * 96 : 0;
  auto a_read = [&](int qd, int s, i32x4& a0, i32x4& a1) {
    const uint8_t* src = lds + a_base + qd * a_qmul + s * 96;
    a0 = *reinterpret_cast<const i32x4*>(src);
    a1 = *reinterpret_cast<const i32x4*>(src + 48);
  };

  // ---- items
  float acc = 0.f;
  float accs[NPW];
#pragma unroll
  for (int i = 0; i < NPW; ++i) accs[i] = 0.f;

  auto item = [&](const ItemPos& x, const Raw<BITS>(&bf)[CPG], uint32_t sraw) {
    const int qd = x.qd;
    if (qd < P) acc = 0.f;  // first quad of this stripe
    i32x4 d = meta[qd * 4 + h];
    const float sE = bf2f(sraw & 0xFFFFu) * __int_as_float(d[3]);
#pragma unroll
    for (int s = 0; s < CPG; ++s) {
      i32x4 b0, b1;
      make_b<BITS>(bf[s], b0, b1);
      i32x4 a0, a1;
      a_read(qd, s, a0, a1);
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
    }
    acc = fmaf(group_sum_f32(d), sE, acc);
    if (qd + P < nquad) return;  // more quads in this stripe
#pragma unroll
    for (int i = 0; i < NPW; ++i)
      if (i == x.ls) accs[i] = acc;
    const int p_next = (x.ls + 1) * SWD + sw;
    if (x.ls + 1 < NPW && p_next < P) return;  // more stripes for this wave
    // row block done for this wave: stripe partials part[p] = ((s0 + s1) + s2) + s3 over the four group slots
    const int rb = x.it * RWV + rw;
    const void* wt;
    const uint16_t* st;
    int n, orow;
    bool ok;
    row_info(rb, wt, st, n, orow, ok);
    float pp[NPW];
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      const float v0 = __shfl(accs[i], r), v1 = __shfl(accs[i], r + 16), v2 = __shfl(accs[i], r + 32),
                  v3 = __shfl(accs[i], r + 48);
      pp[i] = ((v0 + v1) + v2) + v3;
    }
    const int sg = seg_of(sgs, rb * 16);
    if (SWD == 1) {
      float y = pp[0];
#pragma unroll
      for (int i = 1; i < NPW; ++i)
        if (i < P) y += pp[i];
      if (h == 0 && ok) sgs.y[sg][orow] = f2bf(y);
    } else {
      const int il = (x.it - (int)blockIdx.x) / (int)gridDim.x;  // this workgroup's iteration number
      float* slot = part + ((size_t)il * RWV + rw) * 8 * 16;
      if (h == 0) {
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
          const int p = i * SWD + sw;
          if (p < P) slot[p * 16 + r] = pp[i];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      int last = 0;
      if (lane == 0) last = atomicAdd(&tickets[il * RWV + rw], 1) == SWD - 1;
      last = __shfl(last, 0);
      if (last) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (h == 0 && ok) {
          float y = slot[r];
          for (int p = 1; p < P; ++p) y += slot[p * 16 + r];
          sgs.y[sg][orow] = f2bf(y);
        }
      }
    }
  };

  ItemPos pc = pb;
  advance(pc);
  pc.valid = pc.valid && pb.valid;
  while (pa.valid) {
    item(pa, buf0, s0);
    fetch(pc, buf0, s0);
    pa = pc;  // buf0 now holds pc
    if (!pb.valid) break;
    advance(pc);
    pc.valid = pc.valid && pb.valid;
    item(pb, buf1, s1);
    fetch(pc, buf1, s1);
    pb = pc;  // buf1 now holds pc
    advance(pc);
    pc.valid = pc.valid && pa.valid;
  }
  AK_M1_STAMP(3);
}

template <int G>
size_t m1_x_bytes(int nquad) {
  constexpr int CPQ = 4 * G / 32;
  return 512 + (size_t)nquad * (CPQ * 96 + 4 * 16);  // zeros, limbs, meta
}

template <int BITS, int G, int SWD, int NWV>
int launch_m1(I8Args a, hipStream_t s) {
  constexpr int RWV = NWV / SWD;
  const int rows_pad = a.segs.end[a.segs.nseg - 1];
  const int n_rb = rows_pad / 16;
  const int n_iter = (n_rb + RWV - 1) / RWV;
  const size_t x_bytes = m1_x_bytes<G>(a.nquad);
  // workgroups per CU: LDS (160 KB per CU) and waves (NWV each; up to 4 waves per SIMD at <= 128 VGPRs)
  int per_cu = (int)((160 * 1024) / (x_bytes + 4096));
  const int by_waves = 16 / NWV;
  if (per_cu > by_waves) per_cu = by_waves;
  if (per_cu < 1) per_cu = 1;
  int grid = num_cus() * per_cu;
  if (grid > n_iter) grid = n_iter;
  a.iters_max = (n_iter + grid - 1) / grid;
  const size_t smem = x_bytes + (SWD > 1 ? (size_t)a.iters_max * RWV * (8 * 16 * 4 + 4) : 0);
  if (smem > 160 * 1024) return AK_INVALID;
  hipLaunchKernelGGL((i8_m1_kernel<BITS, G, SWD, NWV, 4>), dim3(grid), dim3(64 * NWV), smem, s, a);
  return (int)hipGetLastError();
}

template <int BITS, int G, int NWV>
int m1_swd(const I8Args& a, hipStream_t s) {
  // enough waves to cover the GPU: each row block is shared by SWD stripe-waves (SWD <= P, a power of 2)
  const int n_rb = a.segs.end[a.segs.nseg - 1] / 16;
  const int target = num_cus() * NWV;
  int swd = 1;
  while (swd < 8 && swd * 2 <= a.P && n_rb * swd < target) swd *= 2;
  switch (swd) {
    case 1: return launch_m1<BITS, G, 1, NWV>(a, s);
    case 2: return launch_m1<BITS, G, 2, NWV>(a, s);
    case 4: return launch_m1<BITS, G, 4, NWV>(a, s);
    default: return launch_m1<BITS, G, 8, NWV>(a, s);
  }
}

template <int BITS, int G>
int m1_shape(const I8Args& a, hipStream_t s) {
  // one 16-wave workgroup per CU when two copies of x would fit the LDS (x is converted once per CU, not twice)
  if ((160 * 1024) / (m1_x_bytes<G>(a.nquad) + 4096) >= 2) return m1_swd<BITS, G, 16>(a, s);
  return m1_swd<BITS, G, 8>(a, s);
}

}  // namespace

// one token; segments padded to 16 rows.  Returns 1 if the activation vector does not fit the LDS (caller falls back).
int i8_gemv_m1d(int bits, const void* x, const Segs& g, int k, hipStream_t s);

int i8_gemv_m1(int bits, const void* x, const Segs& g, int k, int group, hipStream_t s) {
  if (group == 128) {
    const int e = i8_gemv_m1d(bits, x, g, k, s);
    if (e != AK_INVALID) return e;
  }
  I8Args a;
  a.segs = g;
  a.x = static_cast<const uint16_t*>(x);
  a.m = 1;
  a.k = k;
  a.nquad = kpad(k) / group / 4;
  a.P = a.nquad < 8 ? a.nquad : 8;
  a.nb = 0;
  a.iters_max = 1;
  switch (bits * 1000 + group) {
    case 4128: return m1_shape<4, 128>(a, s);
    case 3128: return m1_shape<3, 128>(a, s);
    case 2128: return m1_shape<2, 128>(a, s);
    case 4064: return m1_shape<4, 64>(a, s);
    case 3064: return m1_shape<3, 64>(a, s);
    case 2064: return m1_shape<2, 64>(a, s);
    default: return AK_INVALID;
  }
}

}  // namespace agq
