// Default numerics of the mixed-bit GEMV on gfx950: exact integer group dot products on the int8 matrix cores.
//
// Why: at 8 TB/s a W2 / W3 / W4 GEMV streams 32 / 21 / 16 T weights/s, which leaves ~1.2 / 1.8 / 2.4 VALU ops per
// weight on the 256 CUs; a fp32 FMA path spends ~5.  Here every weight costs 1-2 bit operations to become an int8
// matrix operand, and the multiply-adds run on MFMA (v_mfma_i32_16x16x64_i8).
//
// Numerics (restated on the CPU by the test oracle, bit for bit):
//   activations, per (token, group of G inputs): E = the largest bf16 exponent field of the group;
//     x_int = trunc(x * 2^(148 - E)), |x_int| < 2^22, split into three balanced int8 limbs x_int = d2*2^16 + d1*2^8 + d0
//     (d0 = byte 0 of x_int, d1 = byte 1 of x_int + 0x80, d2 = byte 2 of x_int + 0x8080, as signed bytes);
//   weights: the stored code n = q + OFF (OFF = 8 / 4 / 2 for W4 / W3 / W2) as an int8 operand; the MFMA adds
//     sum(d_j * n) - OFF * sum(d_j) (the second term from the same activation operand against a constant -OFF
//     operand), i.e. the exact integer limb sums of sum(d_j * q); GS = combined exactly in fp64;
//     gs = fp32_rn(GS * 2^(E - 148));
//   groups are taken in quads (4 consecutive groups, slot s = g % 4) and the 1024-input tiles in P = min(8, #tiles)
//     contiguous stripes (stripe p = tiles [p * nt / P, (p + 1) * nt / P)); acc[p][s] = fmaf(gs, scale, acc[p][s])
//     over a stripe's quads in order;
//     part[p] = ((acc[p][0] + acc[p][1]) + acc[p][2]) + acc[p][3]; y = part[0] + part[1] + ... left to right; bf16 RN.
// The group sums are exact, so every kernel shape (token count, segmentation, row grouping, bit width of the same
// values) gives the same bits; only the fixed fp32 order above rounds.
//
// MFMA mapping (16x16x64 int8, wave64): B (64 x 16) = weights: lane l holds output row l % 16 and 16 inputs of the
// lane chunk of "lane group" h = l / 16; one MFMA step covers lane chunks 4s .. 4s+3 of a quad (128 inputs), which is
// one g128 group or two g64 groups.  A (16 x 64) = activation limbs: row 4u + j = limb j of token u (g128; 4 tokens
// per MFMA) or of (token u/2, group parity u%2) (g64; 2 tokens per MFMA, lanes of the other parity hold 0).  D lane l:
// output row l % 16, token (g64: token/parity) l / 16, its three limb sums in D[0..2].
//
// Work decomposition (no inter-workgroup communication): a workgroup of SW x RW waves owns RW*R*16 output rows.
// Stripe-wave sw computes stripes sw, sw + SW, ... (one per round); row-subgroup rw covers R row blocks of 16 rows.
// The activations of a batch of a stripe's quads are converted once per workgroup into LDS (shared by the RW waves of
// that stripe) and reused for all the workgroup's rows; the bias sums come from the MFMA in the same batch.  Weights
// stream item by item (item = one quad of one 16-row block) through two register buffers, two items ahead.  Stripe
// partials stay in registers until the last round, meet in LDS, and are added in stripe order.
#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_i8_common.h"

namespace agq {

int num_cus();

namespace {

// LDS layout of a stripe-wave's activation batch:
//   xl[(((qi * CPQ + cq) * 2 + half) * m + token) * 48 + limb * 16 + 4v + b]   (three 16-byte limb rows per token)
//   ex[(qi * 4 + gq) * m + token] = the group's largest bf16 magnitude pattern (act_scale_bits' argument)
// Converts the units (quad qi, group gq, token j) of quads stripe_begin(p) + i0 + qi, qi < nbq; the RW waves of this stripe
// share the work: the LPU = G / 8 lanes of a unit hold 8 consecutive inputs each.
template <int BITS, int G, int RW>
__device__ __forceinline__ void convert_batch(const I8Args& a, int p, int i0, int nbq, int rw, uint8_t* xl, int* ex) {
  constexpr int LPU = G / 8, UPW = 64 / LPU, CPG = G / 32, CPQ = 4 * CPG;
  const int m = a.m, k = a.k, lane = threadIdx.x & 63, sub = lane % LPU;
  const int units = nbq * 4 * m;
  for (int base = rw * UPW; base < units; base += RW * UPW) {
    const int u = base + lane / LPU;
    const bool live = u < units;
    const int qi = live ? u / (4 * m) : 0, rem = live ? u % (4 * m) : 0, gq = rem / m, j = rem % m;
    const int kk = ((stripe_begin(p, a.nquad, a.P, a.qpt) + i0 + qi) * 4 + gq) * G + 8 * sub;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (live && kk < k) v = *reinterpret_cast<const uint4*>(a.x + (size_t)j * k + kk);
    uint32_t t0[8], t1[8], t2[8];
    const int e = group_limbs<LPU>(v, t0, t1, t2);
    if (live) {
      const int eg0 = 8 * sub, cq = gq * CPG + (eg0 >> 5);
      store_limbs<BITS>(xl + ((size_t)(qi * CPQ + cq) * 2 * m + j) * 48, (size_t)m * 48, eg0 & 31, t0, t1, t2);
      if (sub == 0) ex[(qi * 4 + gq) * m + j] = e;
    }
  }
}

// Per (quad, group, token) bias of the limb sums, -OFF * sum(d_j), computed on the MFMA from the converted limbs
// (A against the constant -OFF operand), stored with E as meta[(qi * 4 + gq) * m + token] = {b0, b1, b2, E}.
template <int BITS, int G, int NP, int RW>
__device__ __forceinline__ void bias_batch(const I8Args& a, int nbq, int rw, const uint8_t* xl, const int* ex,
                                           i32x4* meta) {
  constexpr int TPM = G == 128 ? 4 : 2, CPG = G / 32, CPQ = 4 * CPG, SPQ = CPQ / 4;
  const int m = a.m, lane = threadIdx.x & 63, r = lane & 15, h = lane >> 4;
  const int limb_a = r & 3, ua = r >> 2;
  const int tok_a0 = G == 128 ? ua : ua >> 1;
  const bool par_ok = G == 128 ? true : ((ua & 1) == (h >> 1));
  const int tok_d0 = G == 128 ? h : h >> 1, par_d = G == 128 ? 0 : (h & 1);
  const i32x4 negoff = {neg_off_bytes<BITS>(), neg_off_bytes<BITS>(), neg_off_bytes<BITS>(), neg_off_bytes<BITS>()};
  const i32x4 zero = {0, 0, 0, 0};
  const int combos = nbq * SPQ * NP;
  for (int c = rw; c < combos; c += RW) {
    const int qi = c / (SPQ * NP), s = (c / NP) % SPQ, ps = c % NP;
    i32x4 a0 = zero, a1 = zero;
    const int tok_a = ps * TPM + tok_a0;
    if (limb_a < 3 && par_ok && tok_a < m) {
      const uint8_t* src = xl + ((size_t)(qi * CPQ + 4 * s + h) * 2 * m + tok_a) * 48 + 16 * limb_a;
      a0 = *reinterpret_cast<const i32x4*>(src);
      a1 = *reinterpret_cast<const i32x4*>(src + (size_t)m * 48);
    }
    i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, negoff, zero, 0, 0, 0);
    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, negoff, d, 0, 0, 0);
    const int tok_d = ps * TPM + tok_d0, gq = G == 128 ? s : 2 * s + par_d;
    if (r == 0 && tok_d < m) {
      const int idx = (qi * 4 + gq) * m + tok_d;
      i32x4 v = d;
      v[3] = act_scale_bits(ex[idx]);
      meta[idx] = v;
    }
  }
}

// Row block `rbg` (global index of 16 rows) of the concatenated segments: weights, scales, rows, this lane's row
struct RowBlock {
  const void* wt;
  const uint16_t* st;
  int n, orow;
};
__device__ __forceinline__ RowBlock row_block(const Segs& sgs, int rbg, int r, int rows_pad) {
  RowBlock b;
  const int g0 = rbg * 16;
  const int sg = g0 < rows_pad ? seg_of(sgs, g0) : 0;
  b.n = sgs.n[sg];
  const int orow = g0 - (sg ? sgs.end[sg - 1] : 0) + r;
  b.orow = g0 < rows_pad && orow < b.n ? orow : 0;  // padding rows load row 0 of the segment (results unused)
  b.wt = sgs.wt[sg];
  b.st = sgs.st[sg];
  return b;
}

// WPE: waves per SIMD the register allocation must allow (HIP's second launch bound).
// A wave owns R row blocks (R = rows / 16 of the workgroup / RW) for its stripe(s); it streams "items" (quad qi of row
// block j, row-block major) through two register buffers that ping-pong two items ahead.  The accumulators of the
// current row block live in registers; across activation batches they are parked in LDS (accs).
template <int BITS, int G, int NP, int R, int SW, int RW, int WPE>
__global__ void __launch_bounds__(64 * SW * RW, WPE) i8_gemv_kernel(const I8Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int TPM = G == 128 ? 4 : 2;  // tokens per MFMA
  constexpr int CPG = G / 32, CPQ = 4 * CPG, SPQ = CPQ / 4, SPT = 1024 / G;
  constexpr int ROWS = RW * R * 16;
  const int m = a.m, P = a.P, nb = a.nb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sw = wave % SW, rw = wave / SW;
  const int r = lane & 15, h = lane >> 4;
  const Segs& sgs = a.segs;
  const int rows_pad = sgs.end[sgs.nseg - 1];
  const int rb0 = blockIdx.x * RW * R + rw * R;  // this wave's first row block

  // A-operand role of this lane (fixed): token and limb of MFMA row r, and whether its lane group feeds that row
  const int limb_a = r & 3, ua = r >> 2;
  const int tok_a0 = G == 128 ? ua : ua >> 1;
  const bool par_ok = G == 128 ? true : ((ua & 1) == (h >> 1));
  // D role: token (per pass) and group parity (g64) of this lane
  const int tok_d0 = G == 128 ? h : h >> 1, par_d = G == 128 ? 0 : (h & 1);
  const i32x4 zero = {0, 0, 0, 0};

  // LDS: [part: P x ROWS x m floats][per stripe-wave: activation batch, meta, E][accs: parked accumulators]
  const size_t part_bytes = (size_t)P * ROWS * m * 4;
  const size_t xl_bytes = (size_t)nb * CPQ * 2 * m * 48;
  const size_t meta_n = (size_t)nb * 4 * m;
  const size_t wave_bytes = xl_bytes + meta_n * 20;
  float* part = reinterpret_cast<float*>(lds);
  uint8_t* xl = lds + part_bytes + sw * wave_bytes;
  i32x4* meta = reinterpret_cast<i32x4*>(xl + xl_bytes);
  int* ex = reinterpret_cast<int*>(meta + meta_n);
  float* accs = reinterpret_cast<float*>(lds + part_bytes + SW * wave_bytes) + (size_t)wave * R * NP * 4 * 64;

  for (int p0 = 0; p0 < P; p0 += SW) {
    const int p = p0 + sw;
    const int q0 = p < P ? stripe_begin(p, a.nquad, P, a.qpt) : 0;
    const int nq = p < P ? stripe_begin(p + 1, a.nquad, P, a.qpt) - q0 : 0;
    const int nq_round = a.qpt * ((a.nquad / a.qpt + P - 1) / P);  // no stripe has more quads
    for (int i0 = 0; i0 < nq_round; i0 += nb) {
      const int nbq = nq - i0 < nb ? nq - i0 : nb;  // <= 0 when this wave's stripe has no quad here
      const bool last_batch = i0 + nb >= nq;
      const int T = nbq > 0 ? nbq * R : 0;        // items of this batch
      auto fetch = [&](int t, Raw<BITS>(&dst)[SPQ], uint2& sdst) {
        if (t >= T) return;
        const int j = t / nbq, qi = t - j * nbq;
        const RowBlock b = row_block(sgs, rb0 + j, r, rows_pad);
        const int qd = q0 + i0 + qi;
#pragma unroll
        for (int s = 0; s < SPQ; ++s) {
          const int cg = qd * CPQ + 4 * s + h;
          dst[s] = load_raw<BITS>(b.wt, (size_t)(cg >> 5) * b.n + b.orow, cg & 31);
        }
        const int g0 = qd * 4;
        sdst = *reinterpret_cast<const uint2*>(b.st + ((size_t)(g0 / SPT) * b.n + b.orow) * SPT + (g0 % SPT));
      };
      // the first two items are requested before the activations are converted (weights do not depend on them)
      Raw<BITS> buf0[SPQ], buf1[SPQ];
      uint2 sb0, sb1;
      fetch(0, buf0, sb0);
      fetch(1, buf1, sb1);
      __syncthreads();
      if (nbq > 0) convert_batch<BITS, G, RW>(a, p, i0, nbq, rw, xl, ex);
      __syncthreads();
      if (nbq > 0) bias_batch<BITS, G, NP, RW>(a, nbq, rw, xl, ex, meta);
      __syncthreads();
      float acc[NP][4];
      auto item = [&](int t, const Raw<BITS>(&bf)[SPQ], const uint2 s2) {
        const int j = t / nbq, qi = t - j * nbq;
        if (qi == 0) {
#pragma unroll
          for (int ps = 0; ps < NP; ++ps)
#pragma unroll
            for (int s = 0; s < 4; ++s) acc[ps][s] = i0 == 0 ? 0.f : accs[((j * NP + ps) * 4 + s) * 64 + lane];
        }
#pragma unroll
        for (int s = 0; s < SPQ; ++s) {
          const int gq = G == 128 ? s : 2 * s + par_d;  // group in quad of this D lane
          i32x4 b0, b1;
          make_b<BITS>(bf[s], b0, b1);
          const float sc = bf2f((((gq & 2) ? s2.y : s2.x) >> (16 * (gq & 1))) & 0xFFFFu);
#pragma unroll
          for (int ps = 0; ps < NP; ++ps) {
            i32x4 a0 = zero, a1 = zero;
            const int tok_a = ps * TPM + tok_a0;
            if (limb_a < 3 && par_ok && tok_a < m) {
              const uint8_t* src = xl + ((size_t)(qi * CPQ + 4 * s + h) * 2 * m + tok_a) * 48 + 16 * limb_a;
              a0 = *reinterpret_cast<const i32x4*>(src);
              a1 = *reinterpret_cast<const i32x4*>(src + (size_t)m * 48);
            }
            const int tok_d = ps * TPM + tok_d0;
            const i32x4 c = meta[(qi * 4 + gq) * m + (tok_d < m ? tok_d : 0)];
            i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, c, 0, 0, 0);
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
            // g128: slot s; g64: this lane's slots are par_d (s = 0) and par_d + 2 (s = 1), kept at acc[.][s]
            acc[ps][s] = fmaf(group_sum_f32(d), sc * __int_as_float(c[3]), acc[ps][s]);
          }
        }
        if (qi == nbq - 1) {
          if (!last_batch) {
#pragma unroll
            for (int ps = 0; ps < NP; ++ps)
#pragma unroll
              for (int s = 0; s < 4; ++s) accs[((j * NP + ps) * 4 + s) * 64 + lane] = acc[ps][s];
          } else {
#pragma unroll
            for (int ps = 0; ps < NP; ++ps) {
              float s0 = acc[ps][0], s1 = acc[ps][1], s2v = acc[ps][2], s3 = acc[ps][3];
              if (G == 64) {  // this lane holds slots par_d, par_d + 2; the partner lane (h ^ 1) the other parity
                const float mine0 = acc[ps][0], mine2 = acc[ps][1];
                const float oth0 = __shfl_xor(mine0, 16), oth2 = __shfl_xor(mine2, 16);
                s0 = par_d ? oth0 : mine0;
                s1 = par_d ? mine0 : oth0;
                s2v = par_d ? oth2 : mine2;
                s3 = par_d ? mine2 : oth2;
              }
              const int tok = ps * TPM + tok_d0;
              if (tok < m && par_d == 0)
                part[((size_t)p * ROWS + (rw * R + j) * 16 + r) * m + tok] = ((s0 + s1) + s2v) + s3;
            }
          }
        }
      };
      for (int t = 0; t < T; t += 2) {
        item(t, buf0, sb0);
        fetch(t + 2, buf0, sb0);
        if (t + 1 < T) {
          item(t + 1, buf1, sb1);
          fetch(t + 3, buf1, sb1);
        }
      }
    }
  }
  __syncthreads();
  // y = part[0] + part[1] + ... in stripe order
  for (int idx = tid; idx < ROWS * m; idx += 64 * SW * RW) {
    const int rr = idx / m, tok = idx % m;
    const int g = blockIdx.x * ROWS + rr;
    if (g >= rows_pad) continue;
    const int sg = seg_of(sgs, g);
    const int orow = g - (sg ? sgs.end[sg - 1] : 0);
    if (orow >= sgs.n[sg]) continue;
    float v = part[(size_t)rr * m + tok];
    for (int p = 1; p < P; ++p) v += part[((size_t)p * ROWS + rr) * m + tok];
    sgs.y[sg][(size_t)tok * sgs.ldy[sg] + orow] = f2bf(v);
  }
}

constexpr size_t kLdsBudget = 96 * 1024;  // activation batches + partials
constexpr size_t kLdsMax = 160 * 1024;

// LDS bytes of one stripe-wave's batch quad (activation limbs, bias / E meta, E) for m tokens
size_t lds_per_quad(int group, int m) {
  const int cpq = 4 * group / 32;
  return (size_t)m * ((size_t)cpq * 2 * 48 + 4 * 20);
}

template <int BITS, int G, int NP, int R, int SW, int RW, int WPE = 1>
int launch_i8(I8Args a, hipStream_t s) {
  constexpr int ROWS = RW * R * 16;
  const int rows_pad = a.segs.end[a.segs.nseg - 1];
  const size_t per_q = lds_per_quad(G, a.m);
  const size_t part_bytes = (size_t)a.P * ROWS * a.m * 4;
  const size_t accs_bytes = (size_t)SW * RW * R * NP * 4 * 64 * 4;
  const int max_q = a.qpt * ((a.nquad / a.qpt + a.P - 1) / a.P);
  int nb = (int)((kLdsBudget - part_bytes) / (SW * per_q));
  if (nb > max_q) nb = max_q;
  if (nb < 1) return AK_INVALID;
  a.nb = nb;
  const size_t smem = part_bytes + SW * nb * per_q + (nb < max_q ? accs_bytes : 0);
  if (smem > kLdsMax) return AK_INVALID;
  hipLaunchKernelGGL((i8_gemv_kernel<BITS, G, NP, R, SW, RW, WPE>), dim3((rows_pad + ROWS - 1) / ROWS),
                     dim3(64 * SW * RW), smem, s, a);
  return (int)hipGetLastError();
}

// shape by token passes: the LDS of a batch quad grows with m, so fewer stripe-waves (more rounds) for larger m
template <int BITS, int G>
int i8_shape(const I8Args& a, hipStream_t s) {
  constexpr int TPM = G == 128 ? 4 : 2;
  const int np = (a.m + TPM - 1) / TPM;
  if (np <= 1) return launch_i8<BITS, G, 1, 4, 8, 1, 4>(a, s);
  if (np <= 2) return launch_i8<BITS, G, 2, 2, 2, 2>(a, s);
  if (G == 128 || np <= 4) return launch_i8<BITS, G, 4, 1, 1, 2>(a, s);
  if constexpr (G == 64) return launch_i8<BITS, G, 8, 1, 1, 2>(a, s);
  return AK_INVALID;
}

}  // namespace

// 1 <= m <= 16; segments padded to 16 rows.
int i8_gemv(int bits, const void* x, int m, const Segs& g, int k, int group, hipStream_t s) {
  I8Args a;
  a.segs = g;
  a.x = static_cast<const uint16_t*>(x);
  a.m = m;
  a.k = k;
  a.nquad = kpad(k) / group / 4;
  a.qpt = 256 / group;
  a.P = stripe_count(a.nquad, a.qpt);
  a.nb = 1;
  switch (bits * 1000 + group) {
    case 4128: return i8_shape<4, 128>(a, s);
    case 3128: return i8_shape<3, 128>(a, s);
    case 2128: return i8_shape<2, 128>(a, s);
    case 4064: return i8_shape<4, 64>(a, s);
    case 3064: return i8_shape<3, 64>(a, s);
    case 2064: return i8_shape<2, 64>(a, s);
    default: return AK_INVALID;
  }
}

}  // namespace agq
