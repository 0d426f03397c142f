// Default numerics of the mixed-bit GEMV on gfx950: exact integer group dot products on the int8 matrix cores.
//
// Why: at 8 TB/s a W2 / W3 / W4 GEMV streams 32 / 21 / 16 T weights/s, which leaves ~1.2 / 1.8 / 2.4 VALU ops per
// weight on the 256 CUs; a fp32 FMA path spends ~5.  Here every weight costs 1-2 bit operations to become an int8
// matrix operand, and the multiply-adds run on MFMA (v_mfma_i32_16x16x64_i8).
//
// Numerics (restated on the CPU by the test oracle, bit for bit):
//   activations, per (token, group of G inputs): E = the largest bf16 exponent field of the group;
//     x_int = trunc(x * 2^(148 - E)), |x_int| < 2^22, split into three balanced int8 limbs x_int = d2*2^16 + d1*2^8 + d0;
//   weights: the stored code n = q + OFF (OFF = 8 / 4 / 2 for W4 / W3 / W2) as an int8 operand;
//   per (row, token, group): the MFMA accumulates sum(d_j * n) for the three limbs onto an initial -OFF * sum(d_j),
//     giving the exact integer limb sums of sum(d_j * q); GS = combined exactly in fp64; gs = fp32_rn(GS * 2^(E-148));
//   groups are taken in quads (4 consecutive groups, slot s = g % 4) and quads in P = min(8, #quads) stripes
//     (stripe = quad % P); acc[p][s] = fmaf(gs, scale, acc[p][s]) over a stripe's quads in order;
//     part[p] = ((acc[p][0] + acc[p][1]) + acc[p][2]) + acc[p][3]; y = part[0] + part[1] + ... left to right; bf16 RN.
// The group sums are exact, so every kernel shape (token count, segmentation, stripe split, bit width of the same
// values) gives the same bits; only the fixed fp32 order above rounds.
//
// Mapping (16x16x64 int8 MFMA, wave64):  B (64 x 16) = weights: lane l holds output row l % 16 and 16 inputs of the
// lane chunk of "lane group" h = l / 16; one MFMA "step" covers the 4 lane chunks 4s .. 4s+3 of a quad (128 inputs),
// which is one g128 group or two g64 groups.  A (16 x 64) = activation limbs: row 4u + j = limb j of token u (g128;
// 4 tokens per MFMA) or of (token u/2, group parity u%2) (g64; 2 tokens per MFMA, lanes of the other parity hold 0).
// D lane l: row l % 16, token (or token/parity) l / 16, its three limb sums in D[0..2].
//
// Grid: blockIdx.x = 64 output rows (4 waves x 16 rows), blockIdx.y = stripe (split mode) or all stripes (direct
// mode).  Each workgroup converts the activations of its quads into LDS once and reuses them for its 64 rows.  In
// split mode each workgroup writes its stripe partial (fp32) and the last one to finish a row range (atomic ticket)
// adds the P partials in stripe order and writes y; it also resets the ticket, so graphs replay.
#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {

int num_cus();

struct I8Args {
  Segs segs;
  const uint16_t* x;
  int m, k;
  int nquad, P;         // quads of the padded k, stripes
  int nb;               // quads per LDS batch
  float* part;          // split mode: [P][m][rows_pad]
  unsigned* ctr;        // split mode: one ticket per 64-row range
};

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <int BITS>
constexpr int code_offset() { return BITS == 4 ? 8 : BITS == 3 ? 4 : 2; }

// position of input o (0..31) of a lane chunk inside the B operand pair: MFMA half, VGPR v, byte b
template <int BITS>
__device__ __forceinline__ void operand_pos(int o, int& half, int& v, int& b) {
  if (BITS == 4) {  // VGPR v = word v, half 0 = even nibbles, half 1 = odd nibbles
    v = o >> 3, b = (o & 7) >> 1, half = o & 1;
  } else if (BITS == 2) {  // half = word, VGPR s = fields 4b + s
    half = o >> 4, v = o & 3, b = (o & 15) >> 2;
  } else {  // W3: dword t = o % 8 holds inputs 8b + t
    half = (o & 7) >> 2, v = o & 3, b = o >> 3;
  }
}

// B operands (two MFMA halves of 16 int8 codes each) of one lane chunk
template <int BITS>
struct Raw;
template <>
struct Raw<4> { uint4 w; };
template <>
struct Raw<3> { uint2 lo; uint32_t hi; };
template <>
struct Raw<2> { uint2 lo; };

template <int BITS>
__device__ __forceinline__ Raw<BITS> load_raw(const void* __restrict__ wt, size_t rec, int c) {
  Raw<BITS> r;
  if constexpr (BITS == 4) {
    r.w = ld_stream(reinterpret_cast<const uint4*>(wt) + rec * 32 + c);
  } else {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(wt) + rec * (32 * BITS);
    r.lo = ld_stream2(reinterpret_cast<const uint2*>(p) + c);
    if constexpr (BITS == 3) r.hi = ld_stream1(p + 64 + c);
  }
  return r;
}

template <int BITS>
__device__ __forceinline__ void make_b(const Raw<BITS>& r, i32x4& b0, i32x4& b1) {
  if constexpr (BITS == 4) {
    const uint32_t w[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      b0[v] = (int)(w[v] & 0x0F0F0F0Fu);
      b1[v] = (int)((w[v] >> 4) & 0x0F0F0F0Fu);
    }
  } else if constexpr (BITS == 2) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      b0[s] = (int)((r.lo.x >> (2 * s)) & 0x03030303u);
      b1[s] = (int)((r.lo.y >> (2 * s)) & 0x03030303u);
    }
  } else {
    const uint32_t L0 = r.lo.x, L1 = r.lo.y, H = r.hi;
    // bytes m of P0 / P1 hold the 2-bit fields of inputs 8m .. 8m+3 / 8m+4 .. 8m+7
    const uint32_t P0 = (L0 & 0xFFu) | ((L0 >> 8) & 0xFF00u) | ((L1 & 0xFFu) << 16) | ((L1 << 8) & 0xFF000000u);
    const uint32_t P1 = ((L0 >> 8) & 0xFFu) | ((L0 >> 16) & 0xFF00u) | ((L1 << 8) & 0xFF0000u) | (L1 & 0xFF000000u);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      b0[t] = (int)(((P0 >> (2 * t)) & 0x03030303u) | (((H >> t) & 0x01010101u) << 2));
      b1[t] = (int)(((P1 >> (2 * t)) & 0x03030303u) | (((H >> (t + 4)) & 0x01010101u) << 2));
    }
  }
}

__device__ __forceinline__ float combine_limbs(const i32x4& d, int E) {
  const double g = ((double)d[2] * 65536.0 + (double)d[1] * 256.0) + (double)d[0];  // exact (< 2^53)
  return (float)ldexp(g, E - 148);
}

// Convert the activations of `nbq` quads of stripe p (quads p + (i0 + qi) * P) into LDS:
//   xl[((((qi * CPQ + cq) * 2 + half) * m + token) * 3 + limb) * 16 + 4v + b] = limb byte of that input,
//   meta[(qi * 4 + gq) * m + token] = {-OFF * sum d0, -OFF * sum d1, -OFF * sum d2, E}.
template <int BITS, int G>
__device__ __forceinline__ void convert_x(const I8Args& a, int p, int i0, int nbq, uint8_t* xl, i32x4* meta) {
  constexpr int LPU = G / 8;  // lanes per group, 8 inputs per lane
  constexpr int CPG = G / 32, CPQ = 4 * CPG;
  constexpr int OFF = code_offset<BITS>();
  const int m = a.m, k = a.k;
  const int tid = threadIdx.x, sub = tid % LPU;
  const int units = nbq * 4 * m;
  for (int u = tid / LPU; u < ((units + kThreads / LPU - 1) / (kThreads / LPU)) * (kThreads / LPU);
       u += kThreads / LPU) {
    const bool live = u < units;
    const int qi = live ? u / (4 * m) : 0, rem = live ? u % (4 * m) : 0, gq = rem / m, j = rem % m;
    const int qd = p + (i0 + qi) * a.P;
    const int kk = (qd * 4 + gq) * G + 8 * sub;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (live && kk < k) v = *reinterpret_cast<const uint4*>(a.x + (size_t)j * k + kk);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    int e = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) e = max(e, max((int)((w[i] >> 7) & 0xFFu), (int)((w[i] >> 23) & 0xFFu)));
#pragma unroll
    for (int o = 1; o < LPU; o <<= 1) e = max(e, __shfl_xor(e, o));
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t bits16 = (w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      const int xi = (int)ldexpf(bf2f(bits16), 148 - e);  // exact; truncation toward zero
      const int x1 = (xi + 128) >> 8, x2 = (x1 + 128) >> 8;
      const int d0 = xi - (x1 << 8), d1 = x1 - (x2 << 8);
      s0 += d0, s1 += d1, s2 += x2;
      const int eg = 8 * sub + i, cq = gq * CPG + (eg >> 5);
      int half, vv, bb;
      operand_pos<BITS>(eg & 31, half, vv, bb);
      if (live) {
        uint8_t* dst = xl + ((((size_t)qi * CPQ + cq) * 2 + half) * m + j) * 48 + 4 * vv + bb;
        dst[0] = (uint8_t)d0;
        dst[16] = (uint8_t)d1;
        dst[32] = (uint8_t)x2;
      }
    }
#pragma unroll
    for (int o = 1; o < LPU; o <<= 1) {
      s0 += __shfl_xor(s0, o);
      s1 += __shfl_xor(s1, o);
      s2 += __shfl_xor(s2, o);
    }
    if (live && sub == 0) {
      i32x4 mv;
      mv[0] = -OFF * s0, mv[1] = -OFF * s1, mv[2] = -OFF * s2, mv[3] = e;
      meta[(qi * 4 + gq) * m + j] = mv;
    }
  }
}

template <int BITS, int G, int NP>
__global__ void __launch_bounds__(kThreads) i8_gemv_kernel(const I8Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int TPM = G == 128 ? 4 : 2;  // tokens per MFMA
  constexpr int CPG = G / 32, CPQ = 4 * CPG, SPQ = CPQ / 4, SPT = 1024 / G;
  const int m = a.m, P = a.P;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, h = lane >> 4;
  const Segs& sgs = a.segs;
  const int rows_pad = sgs.end[sgs.nseg - 1];
  const int rb = blockIdx.x * kWaves + wave;
  const bool wave_on = rb * 16 < rows_pad;
  int sg = 0, orow = 0, n = 1;
  if (wave_on) {
    sg = seg_of(sgs, rb * 16);
    n = sgs.n[sg];
    orow = rb * 16 - (sg ? sgs.end[sg - 1] : 0) + r;
  }
  const bool row_ok = wave_on && orow < n;
  const int oc = row_ok ? orow : 0;
  const void* wt = sgs.wt[sg];
  const uint16_t* st = sgs.st[sg];

  // A-operand role of this lane (fixed): token and limb of MFMA row r, and whether its lane group feeds that row
  const int limb_a = r & 3, ua = r >> 2;
  const int tok_a0 = G == 128 ? ua : ua >> 1;
  const bool par_ok = G == 128 ? true : ((ua & 1) == (h >> 1));
  // D role: token (per pass) and group-in-step of this lane
  const int tok_d0 = G == 128 ? h : h >> 1, par_d = G == 128 ? 0 : (h & 1);

  const int nb = a.nb;
  uint8_t* xl = lds;
  i32x4* meta = reinterpret_cast<i32x4*>(lds + (size_t)nb * CPQ * 2 * m * 48);

  const bool direct = gridDim.y == 1;
  const int p_first = gridDim.y == 1 ? 0 : blockIdx.y, p_last = gridDim.y == 1 ? P - 1 : blockIdx.y;
  float yv[NP];
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) yv[ps] = 0.f;

  for (int p = p_first; p <= p_last; ++p) {
    const int nq = (a.nquad - p + P - 1) / P;
    float acc[NP][4];
#pragma unroll
    for (int ps = 0; ps < NP; ++ps)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[ps][s] = 0.f;
    for (int i0 = 0; i0 < nq; i0 += nb) {
      const int nbq = nq - i0 < nb ? nq - i0 : nb;
      __syncthreads();
      convert_x<BITS, G>(a, p, i0, nbq, xl, meta);
      __syncthreads();
      if (!wave_on) continue;
      for (int qi = 0; qi < nbq; ++qi) {
        const int qd = p + (i0 + qi) * P;
        Raw<BITS> raw[SPQ];
#pragma unroll
        for (int s = 0; s < SPQ; ++s) {
          const int cg = qd * CPQ + 4 * s + h;
          raw[s] = load_raw<BITS>(wt, (size_t)(cg >> 5) * n + oc, cg & 31);
        }
        // the 4 scales of the quad's groups for row oc (contiguous: a quad never straddles a tile)
        const int g0 = qd * 4;
        const uint2 sw = *reinterpret_cast<const uint2*>(st + ((size_t)(g0 / SPT) * n + oc) * SPT + (g0 % SPT));
        const float scl[4] = {bf2f(sw.x & 0xFFFFu), bf2f(sw.x >> 16), bf2f(sw.y & 0xFFFFu), bf2f(sw.y >> 16)};
#pragma unroll
        for (int s = 0; s < SPQ; ++s) {
          i32x4 b0, b1;
          make_b<BITS>(raw[s], b0, b1);
          const int gq = G == 128 ? s : 2 * s + par_d;  // group in quad of this D lane (meta index)
#pragma unroll
          for (int ps = 0; ps < NP; ++ps) {
            i32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
            const int tok_a = ps * TPM + tok_a0;
            if (limb_a < 3 && par_ok && tok_a < m) {
              const uint8_t* src = xl + (((size_t)qi * CPQ + 4 * s + h) * 2 * m + tok_a) * 48 + 16 * limb_a;
              a0 = *reinterpret_cast<const i32x4*>(src);
              a1 = *reinterpret_cast<const i32x4*>(src + (size_t)m * 48);
            }
            const int tok_d = ps * TPM + tok_d0;
            const i32x4 c = meta[(qi * 4 + gq) * m + (tok_d < m ? tok_d : 0)];
            i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, c, 0, 0, 0);
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
            const float gs = combine_limbs(d, c[3]);
            // g128: slot s; g64: this lane's slots are par_d (s = 0) and par_d + 2 (s = 1), kept at acc[ps][s]
            const float sc = G == 128 ? scl[s] : (par_d ? scl[2 * s + 1] : scl[2 * s]);
            acc[ps][s] = fmaf(gs, sc, acc[ps][s]);
          }
        }
      }
    }
    if (!wave_on) continue;
#pragma unroll
    for (int ps = 0; ps < NP; ++ps) {
      float s0 = acc[ps][0], s1 = acc[ps][1], s2 = acc[ps][2], s3 = acc[ps][3];
      if (G == 64) {  // this lane holds slots par_d, par_d + 2; the partner lane (h ^ 1) the other parity
        const float mine0 = acc[ps][0], mine2 = acc[ps][1];
        const float oth0 = __shfl_xor(mine0, 16), oth2 = __shfl_xor(mine2, 16);
        s0 = par_d ? oth0 : mine0;
        s1 = par_d ? mine0 : oth0;
        s2 = par_d ? oth2 : mine2;
        s3 = par_d ? mine2 : oth2;
      }
      const float part = ((s0 + s1) + s2) + s3;
      if (direct) {
        yv[ps] = p == p_first ? part : yv[ps] + part;
      } else {
        const int tok = ps * TPM + tok_d0;
        if (tok < m && par_d == 0)
          a.part[((size_t)p * m + tok) * rows_pad + rb * 16 + r] = part;
      }
    }
  }

  if (direct) {
    if (row_ok) {
#pragma unroll
      for (int ps = 0; ps < NP; ++ps) {
        const int tok = ps * TPM + tok_d0;
        if (tok < m && par_d == 0) sgs.y[sg][(size_t)tok * sgs.ldy[sg] + orow] = f2bf(yv[ps]);
      }
    }
    return;
  }
  // split mode: the last workgroup of this row range adds the stripe partials in order
  __shared__ int last;
  __threadfence();
  __syncthreads();
  if (tid == 0) last = atomicAdd(a.ctr + blockIdx.x, 1u) == (unsigned)(P - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (row_ok) {
#pragma unroll
    for (int ps = 0; ps < NP; ++ps) {
      const int tok = ps * TPM + tok_d0;
      if (tok < m && par_d == 0) {
        const float* pp = a.part + (size_t)tok * rows_pad + rb * 16 + r;
        float v = __builtin_nontemporal_load(pp);
        for (int p = 1; p < P; ++p) v += __builtin_nontemporal_load(pp + (size_t)p * m * rows_pad);
        sgs.y[sg][(size_t)tok * sgs.ldy[sg] + orow] = f2bf(v);
      }
    }
  }
  if (tid == 0) a.ctr[blockIdx.x] = 0u;
}

template <int BITS, int G, int NP>
int launch_i8(const I8Args& a, int ranges, int split, size_t smem, hipStream_t s) {
  hipLaunchKernelGGL((i8_gemv_kernel<BITS, G, NP>), dim3(ranges, split ? a.P : 1), dim3(kThreads), smem, s, a);
  return (int)hipGetLastError();
}

template <int BITS, int G>
int i8_np(const I8Args& a, int ranges, int split, size_t smem, hipStream_t s) {
  constexpr int TPM = G == 128 ? 4 : 2;
  const int np = (a.m + TPM - 1) / TPM;
  if (np <= 1) return launch_i8<BITS, G, 1>(a, ranges, split, smem, s);
  if (np <= 2) return launch_i8<BITS, G, 2>(a, ranges, split, smem, s);
  if (np <= 4) return launch_i8<BITS, G, 4>(a, ranges, split, smem, s);
  return launch_i8<BITS, G, 8>(a, ranges, split, smem, s);
}

}  // namespace

// LDS bytes per quad for m tokens
size_t i8_lds_per_quad(int group, int m) {
  const int cpq = 4 * group / 32;
  return (size_t)m * (cpq * 2 * 48 + 4 * 16);
}

// 1 <= m <= 16; segments padded to 16 rows.  part / ctr: split-K scratch, or nullptr for direct mode.
int i8_gemv(int bits, const void* x, int m, const Segs& g, int k, int group, float* part, unsigned* ctr,
            hipStream_t s) {
  I8Args a;
  a.segs = g;
  a.x = static_cast<const uint16_t*>(x);
  a.m = m;
  a.k = k;
  a.nquad = kpad(k) / group / 4;
  a.P = a.nquad < 8 ? a.nquad : 8;
  const int max_q = (a.nquad + a.P - 1) / a.P;
  const size_t per_q = i8_lds_per_quad(group, m);
  int nb = (int)((48 * 1024) / per_q);
  if (nb < 1) nb = 1;
  if (nb > max_q) nb = max_q;
  a.nb = nb;
  a.part = part;
  a.ctr = ctr;
  const int rows_pad = g.end[g.nseg - 1];
  const int ranges = (rows_pad + 16 * kWaves - 1) / (16 * kWaves);
  const int split = (part && ctr && a.P > 1) ? 1 : 0;
  const size_t smem = (size_t)nb * per_q;
  switch (bits * 1000 + group) {
    case 4128: return i8_np<4, 128>(a, ranges, split, smem, s);
    case 3128: return i8_np<3, 128>(a, ranges, split, smem, s);
    case 2128: return i8_np<2, 128>(a, ranges, split, smem, s);
    case 4064: return i8_np<4, 64>(a, ranges, split, smem, s);
    case 3064: return i8_np<3, 64>(a, ranges, split, smem, s);
    case 2064: return i8_np<2, 64>(a, ranges, split, smem, s);
    default: return AK_INVALID;
  }
}

}  // namespace agq
