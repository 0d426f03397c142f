// The fp16-MFMA GEMV for more than one token (speculative verify, batched decode), group 128, on gfx950: the route of
// ak_wq_gemv_kt_multi above its measured crossover in m (the role of the reference's tensor-core kernels for m > 1,
// kernels/src/w4_gemv.cu:990-1163: bf16 MMA over the expanded codes, fp32 accumulation).
//
// Numerics: the default numerics of the integer-limb kernels (wq_i8_common.h), bit for bit, so that a token's outputs
// are the same whichever kernel a launch takes and however many tokens share it (the reference's contract for batched
// rows, w4_gemv.cu:1075-1079).  Per (token, group): E = the group's largest bf16 exponent field, x_int =
// trunc(x * 2^(148 - E)) (|x_int| < 2^22), entered into v_mfma_f32_16x16x32_f16 as two exact fp16 limbs, hi = x_int >> 11
// in [-2048, 2048) and lo = x_int & 2047; a stored code n enters as the exact fp16 q = (1024 + n) - (1024 + OFF)
// (OFF = 8 / 4 / 2: one byte permute, bit pattern 0x6400 | n, and one packed fp16 subtraction per pair of codes).
// Every product and partial sum of a group is an integer below 2^21, so each limb's chain of four MFMAs gives its
// exact integer sum, and gsum = fmaf(D_hi, 2048, D_lo) = fp32_rn(sum(x_int * q)), the integer kernels' group sum.
// Then acc[s] = fmaf(gsum, scale * 2^(E - 148), acc[s]) with s = the group's slot in its quad (g mod 4), a stripe's
// partial = ((acc[0] + acc[1]) + acc[2]) + acc[3], stripes P = min(8, #tiles) contiguous runs of whole 1024-input
// tiles, y = stripe partials added left to right, bf16 RNE.  A group holding an Inf or NaN: as the integer kernels
// (act_scale_bits, x_int).
//
// MFMA layout (16-row blocks, one group of 128 inputs per chain of four MFMAs, 16 tokens per token tile):
//   A = activations: lane (c, h) = (lane % 16, lane / 16) holds token c of the tile, slots 8 h .. 8 h + 7 of the k-step;
//   B = weights: lane (c, h) holds output row c, chunk h of the group (32 inputs; k-step j takes 8 of them);
//   D: lane (c, h) holds tokens 4 h + i (i < 4) of the tile for row c.
// k-step j, slot e of lane chunk h is input 32 h + mm_pos<BITS>(j, e) of the group (the order the byte permutes leave
// the codes in); the activation image in LDS holds the inputs in the same order, 16 bytes per (group, k-step, chunk,
// token), so an A operand is one 16-byte LDS read and a 16-lane pass reads 256 contiguous bytes.
//
// Loads and items as the tokens-in-A-rows kernel (wq_i8mt.hip): an item is 16 rows x one quad, whole 128-byte lines
// per row and load instruction pair, one permlane16 swap per dword pair for W2 / W3.
//
// Work decomposition: one persistent workgroup per CU owns a contiguous range of 16-row blocks of one segment; wave w
// owns NBW blocks per round (blocks w + W (NBW rd + b), W waves: 16 for up to 16 tokens, 8 above) and walks the quads
// of its k range in order, the NBW blocks of a quad one after the other, with two items in flight.  The activation image covers a chunk of
// cq quads at a time (all tokens); with more than one chunk the workgroup meets at a barrier, restages, and meets
// again.  SK (split-K across workgroups, one segment, few rows per CU): workgroup (r, p) computes stripe p of row range
// r; stripe partials go to scratch with device-coherent stores and the range's last workgroup adds them in stripe
// order.
#include <type_traits>

#include "agens_kernels.h"
#include "wq_common.h"
#include "wq_i8_common.h"
#include "wq_quad.h"

namespace agq {

int num_cus();
void* stream_scratch(hipStream_t s, size_t bytes);

namespace {

constexpr int kG = 128;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, dword 3 (CDNA)
constexpr int kNt = 2;                    // streaming (non-temporal) cache policy for the weights
constexpr int kVmcnt0 = 0x0F70;            // s_waitcnt immediate: vector memory counter 0, the others unconstrained
constexpr int kMaxTok = 32;               // tokens per launch (2 token tiles: two limb images of 64 tokens leave no room
                                          // for two quads in the LDS)
constexpr size_t kLds = 160 * 1024;
constexpr int kZeros = 1024;  // LDS bytes of zeros at the start: A and C operands of a dummy item

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MmArgs {
  Segs segs;
  const uint16_t* x;
  int m, k;
  int nquad, P;   // quads of the padded k, stripes
  int tl;         // tokens per (group, k-step, chunk) row of the image: 4, 8 or 16 (one tile), 16 per tile above
  int cq;         // quads per chunk of the activation image
  int wg_end[4];  // workgroups of segments 0..i
  float* part;    // SK: stripe partials [P][16-row blocks][16 NTT tokens][16 rows] per segment, and one counter per row range
  int* cnt;
  int act;        // 1: x is the merged gate_up [m][2k] and the activations are SiLU(gate) * up (wq_silu.h)
};

// slot e of k-step j of a lane chunk -> input of the chunk (the order mm_b leaves the codes in)
template <int BITS>
__host__ __device__ constexpr int mm_pos(int j, int e) {
  return BITS == 4 ? 8 * j + (e < 4 ? 2 * e : 2 * (e - 4) + 1)
       : BITS == 2 ? j + 4 * e
                   : j + (e < 4 ? 8 * e : 8 * (e - 4) + 4);
}

// the fp16 pair (q, q') of the byte permute's result (1024 + n, 1024 + n'): one packed subtraction, exact
template <int OFF>
__device__ __forceinline__ uint32_t q_pair(uint32_t v) {
  constexpr _Float16 c = (_Float16)(1024 + OFF);
  f16x2 h;
  __builtin_memcpy(&h, &v, 4);
  h = h - f16x2{c, c};
  uint32_t r;
  __builtin_memcpy(&r, &h, 4);
  return r;
}

// the B operand of k-step j from the group's int8 code operands (make_b): bytes m, m + 1 of a code dword become the
// fp16 pair (q, q'), via 0x6400 | n (a v_perm with the constant 0x64 bytes).  (The codes as the subnormal fp16 n * 2^-24,
// without the subtraction, were measured on this GPU to lose precision in the MFMA: relative error 2.6e-4 of a
// 32-input product sum against exact sums with normal operands.)
template <int BITS>
__device__ __forceinline__ f16x8 mm_b(const i32x4& b0, const i32x4& b1, int j) {
  constexpr uint32_t kHi = 0x64646464u, kS01 = 0x04010400u, kS23 = 0x04030402u;
  constexpr int OFF = code_offset<BITS>();
  const uint4 v = make_uint4(q_pair<OFF>(__builtin_amdgcn_perm(kHi, (uint32_t)b0[j], kS01)),
                             q_pair<OFF>(__builtin_amdgcn_perm(kHi, (uint32_t)b0[j], kS23)),
                             q_pair<OFF>(__builtin_amdgcn_perm(kHi, (uint32_t)b1[j], kS01)),
                             q_pair<OFF>(__builtin_amdgcn_perm(kHi, (uint32_t)b1[j], kS23)));
  f16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// waves per workgroup: 16 for one token tile; 8 for more (their accumulators need the registers of two waves)
template <int NTT>
constexpr int mm_waves() { return NTT == 1 ? 16 : 8; }

template <int BITS, int NTT, int NBW, bool SK, int TL>
__global__ void __launch_bounds__(mm_waves<NTT>() * 64, 1) mm_kernel(const MmArgs a) {
  constexpr int NWV = mm_waves<NTT>();
  static_assert(NTT == 1 ? (TL == 4 || TL == 8 || TL == 16) : TL == 16 * NTT, "token stride of the image");
  extern __shared__ __attribute__((aligned(256))) uint8_t lds[];
  constexpr int REC = 128 * BITS, MP = 16 * NTT;
  static_assert(NBW == 1 || NBW == 2, "one or two blocks per wave and round");
  constexpr int U = 2;  // items per loop step (two in flight)
  constexpr int tl = TL;
  const int P = a.P, nquad = a.nquad, k = a.k, m = a.m, cq = a.cq;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, h = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Segs& sgs = a.segs;

  // this workgroup's segment and its 16-row blocks [b_lo, b_lo + nb) of that segment (SK: row range r, stripe psk)
  const int bid = (int)blockIdx.x;
  int sg = 0;
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) sg += (i < sgs.nseg && bid >= a.wg_end[i - 1]) ? 1 : 0;
  const int wg0 = sg ? AK_PICK(sg - 1, a.wg_end) : 0, li = bid - wg0;
  const int nr = SK ? (AK_PICK(sg, a.wg_end) - wg0) / P : 1, r = SK ? li / P : 0, psk = SK ? li - r * P : 0;
  const int gs = SK ? nr : AK_PICK(sg, a.wg_end) - wg0, w = SK ? r : li;
  const int n = AK_PICK(sg, sgs.n), n_b16 = (n + 15) >> 4;
  const int b_lo = (int)((unsigned)w * (unsigned)n_b16 / (unsigned)gs);
  const int nb = (int)((unsigned)(w + 1) * (unsigned)n_b16 / (unsigned)gs) - b_lo;
  const int ldy = AK_PICK(sg, sgs.ldy);
  uint16_t* const yseg = AK_PICK(sg, sgs.y);
  float* spart = a.part;
  int* scnt = a.cnt;
  if constexpr (SK) {
#pragma unroll
    for (int i = 0; i < kMaxSegs - 1; ++i)
      if (i < sg) spart += (size_t)P * MP * ((AK_PICK(i, sgs.n) + 15) >> 4) * 16;
    scnt += wg0 / P + r;
  }

  // k range: stripes [pa, pb), quads [qa, qb), in chunks of cq quads
  const int pa = SK ? psk : 0, pb = SK ? psk + 1 : P;
  const int qa = stripe_begin(pa, nquad, P, 2), qb = stripe_begin(pb, nquad, P, 2);
  const int nch = (qb - qa + cq - 1) / cq;
  // bit q - qa set when quad q is the last of its stripe (at most 128 quads)
  unsigned long long ends0 = 0, ends1 = 0;
  for (int p = pa; p < pb; ++p) {
    const int e = stripe_begin(p + 1, nquad, P, 2) - 1 - qa;
    if (e < 64) ends0 |= 1ull << e;
    else ends1 |= 1ull << (e - 64);
  }
  // stripe of quad q (relative rq = q - qa): pa + the stripe ends before it
  auto stripe_of = [&](int rq) {
    const unsigned long long m0 = rq >= 64 ? ends0 : (ends0 & ((1ull << rq) - 1ull));
    const unsigned long long m1 = rq <= 64 ? 0ull : (ends1 & ((1ull << (rq - 64)) - 1ull));
    return pa + __builtin_popcountll(m0) + __builtin_popcountll(m1);
  };

  // LDS: zeros [kZeros B: the operands of dummy items] | image [cq * 4 groups][2 limbs][4 k-steps][4 chunks][tl tokens] x 16 B
  //      (fp16) | meta [cq * 4 groups][tl tokens]: the activation scale (fp32 bits)
  //      | outputs [nb][MP tokens][16 rows]: bf16 results (SK: fp32 stripe partials), written out after the loop (a
  //        global store among the streaming loads would make the compiler drain every load in flight)
  const int ls = 16 * tl * 16, gbytes = 2 * ls;  // one limb's image of a group, both limbs
  uint8_t* const img = lds + kZeros;
  float* const meta = reinterpret_cast<float*>(img + (size_t)cq * 4 * gbytes);
  uint8_t* const outl = reinterpret_cast<uint8_t*>(meta + cq * 4 * tl);

  // ---- the activation image of chunk ch: per (token t, group g, chunk hh) one lane loads the 32 inputs and writes
  // them as scaled fp16 in the operand order; the group's scale exponent from its four lanes; padding past k: zeros
  auto stage = [&](int ch) __attribute__((always_inline)) {
    const int q0 = qa + ch * cq, cg = 4 * ((qb - q0 < cq ? qb - q0 : cq));
    // units: per (group g, 16-token block tb) one wave-sized set of 64 lanes, lane = (chunk hh = lane / 16, token
    // tb * 16 + lane % 16): 16 consecutive lanes write 16 consecutive 16-byte token rows of the image (no LDS bank
    // conflicts); the group's exponent over its four chunk lanes (16 and 32 lanes apart) by lane exchanges
    const int ntb = (m + 15) >> 4, units = cg * ntb * 64, xk = a.act ? 2 * k : k;  // x's token stride
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.x), (short)0, m * xk * 2, kRsrcWord3);
    for (int u = tid; u < units; u += blockDim.x) {
      const int hh = (u >> 4) & 3, gi = u >> 6, tb = gi / cg, g = gi - tb * cg, t = tb * 16 + (u & 15);
      const bool tv = t < m;
      const int i0 = (4 * q0 + g) * kG + 32 * hh;  // first input of the lane chunk
      const int xo = ((tv ? t : 0) * xk + (i0 < k ? i0 : 0)) * 2;
      uint32_t X[16];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const u32x4 d = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16 * v, 0, 0);
        uint4 x4 = make_uint4(d[0], d[1], d[2], d[3]);
        if (a.act) {  // SiLU(gate) * up, the up half k inputs further
          const u32x4 e = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 2 * k + 16 * v, 0, 0);
          x4 = silu_mul8(x4, make_uint4(e[0], e[1], e[2], e[3]));
        }
        X[4 * v] = i0 < k ? x4.x : 0u;
        X[4 * v + 1] = i0 < k ? x4.y : 0u;
        X[4 * v + 2] = i0 < k ? x4.z : 0u;
        X[4 * v + 3] = i0 < k ? x4.w : 0u;
      }
      // the group's largest magnitude pattern (NaN / Inf order above every finite one), over the group's four lanes
      uint32_t mx = 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t w = X[i] & 0x7FFF7FFFu;
        mx = max(mx, max(w & 0xFFFFu, w >> 16));
      }
      int mxi = (int)mx;
      mxi = max(mxi, __shfl_xor(mxi, 16));
      mxi = max(mxi, __shfl_xor(mxi, 32));
      const XiScale xs = xi_scale(mxi >> 7);
      uint8_t* dst = img + (size_t)g * gbytes + ((size_t)hh * tl + t) * 16;
      // x_int of each input in the operand order, as its two exact fp16 limbs: hi = x_int >> 11 in [-2048, 2048) (image
      // 0), lo = x_int & 2047 (image 1, ls bytes further)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t dh[4], dl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int i0 = mm_pos<BITS>(j, 2 * q), i1 = mm_pos<BITS>(j, 2 * q + 1);
          const int x0 = x_int((X[i0 >> 1] >> (16 * (i0 & 1))) & 0xFFFFu, xs);
          const int x1 = x_int((X[i1 >> 1] >> (16 * (i1 & 1))) & 0xFFFFu, xs);
          const auto hp = __builtin_amdgcn_cvt_pkrtz((float)(x0 >> 11), (float)(x1 >> 11));
          const auto lp = __builtin_amdgcn_cvt_pkrtz((float)(x0 & 2047), (float)(x1 & 2047));
          __builtin_memcpy(&dh[q], &hp, 4);
          __builtin_memcpy(&dl[q], &lp, 4);
        }
        if (tv) {
          *reinterpret_cast<uint4*>(dst + (size_t)j * 4 * tl * 16) = make_uint4(dh[0], dh[1], dh[2], dh[3]);
          *reinterpret_cast<uint4*>(dst + ls + (size_t)j * 4 * tl * 16) = make_uint4(dl[0], dl[1], dl[2], dl[3]);
        }
      }
      if (tv && hh == 0) reinterpret_cast<int*>(meta)[g * tl + t] = act_scale_bits(mxi);  // 2^(E - 148), NaN, Inf
    }
  };

  // ---- weight addressing (as wq_i8mt.hip): per lane fixed, per item scalar.  Rows past the segment's end read other
  // rows or, past the buffer, zeros; their results are not written.
  const int ntile = nquad >> 1;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(AK_PICK(sg, sgs.wt)), (short)0, ntile * n * REC, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(AK_PICK(sg, sgs.st)), (short)0, ntile * n * 16, kRsrcWord3);
  // pair loads (quad_vo_w / quad_vo_h): whole lines per instruction, each lane's own row after quad_pair_rows
  const int vo_w = quad_vo_w(BITS, c, h, REC), vo_h = quad_vo_h(c, h, REC), vo_s = c * 16;
  const int tile_w = n * REC, tile_s = n * 16;
  auto fetch1 = [&](int blk, int qd, QuadRaw<BITS>& d) __attribute__((always_inline)) {
    const int row0 = (b_lo + blk) * 16, odd = qd & 1;
    const int so = row0 * REC + (qd >> 1) * tile_w;
    if constexpr (BITS == 4) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
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

  // ---- this wave's item sequence: rounds rd, chunks ch, quads q of the chunk, blocks b < NBW (padded per chunk to a
  // multiple of U items); an item past the wave's blocks or the chunk's quads is a dummy: it loads quad qa of block
  // 0 (cache-resident) and is not computed
  const int nrounds = (nb + NWV * NBW - 1) / (NWV * NBW);
  auto seg_items = [&](int ch) {
    const int q0 = qa + ch * cq, nq = qb - q0 < cq ? qb - q0 : cq;
    return (nq * NBW + U - 1) / U * U;
  };
  int frd = 0, fch = 0, fi = 0;
  auto fetch_next = [&](QuadRaw<BITS>& dst) __attribute__((always_inline)) {
    const int q = qa + fch * cq + fi / NBW, bl = wave + NWV * (NBW * frd + fi % NBW);
    const int q1 = qa + fch * cq + (qb - qa - fch * cq < cq ? qb - qa - fch * cq : cq);
    const bool in = frd < nrounds && q < q1 && bl < nb;
    fetch1(in ? bl : 0, in ? q : qa, dst);
    if (++fi == seg_items(fch)) {
      fi = 0;
      if (++fch == nch) fch = 0, ++frd;
    }
  };

  // accumulators per (block, token tile, group slot s = group mod 4 of the quad, output element)
  float acc[NBW][NTT][4][4], yrun[NBW][NTT][4];
#pragma unroll
  for (int b = 0; b < NBW; ++b)
#pragma unroll
    for (int t = 0; t < NTT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        yrun[b][t][i] = 0.f;
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) acc[b][t][sl][i] = 0.f;
      }

  // A operand and C (meta) offsets of this lane: token c of a tile (a one-tile image narrower than 16 tokens: rows past
  // it read token 0, their results are not written)
  const int a_tok = c < tl ? c : 0, m_tok = 4 * h < tl ? 4 * h : 0;

  // one item: block b (compile-time), quad q, chunk's first quad q0, local block bl.  A dummy item (ok = false: the
  // second block of a wave that has one) reads its A and C operands from the zeros, so that it adds exactly zero.  At a stripe end the partial (SK) or, at the
  // last stripe, the output is staged in LDS (no global access here: the loads stay exactly counted).
  auto core = [&](QuadRaw<BITS>& bf, auto bc, int q, int q0, bool ok, int bl) __attribute__((always_inline)) {
    constexpr int b = decltype(bc)::value;
    float sc[4];
    sc[0] = __uint_as_float(bf.s.x << 16);
    sc[1] = __uint_as_float(bf.s.x & 0xFFFF0000u);
    sc[2] = __uint_as_float(bf.s.y << 16);
    sc[3] = __uint_as_float(bf.s.y & 0xFFFF0000u);
    quad_pair_rows<BITS>(bf, (c & 1) != 0);  // in place: the buffer is refilled after the item
    Raw<BITS> rg[4];
    quad_groups<BITS>(bf, rg);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (NTT == 1 && s == 2) asm volatile("" ::: "memory");  // one tile: two groups' operands live at a time
      i32x4 b0, b1;
      make_b<BITS>(rg[s], b0, b1);
      constexpr int tlr = TL;
      const int g = 4 * (q - q0) + s;  // group of the chunk's image
      // (a dummy item -- two blocks per wave only -- reads its operands from the zeros: k-step strides of zero)
      const bool dz = NBW == 2 && !ok;
      const int jst = dz ? 0 : 4 * TL * 16;
      const uint8_t* ab = dz ? lds + lane * 16 : img + (size_t)g * 2 * 256 * tlr + ((size_t)h * tlr + a_tok) * 16;
      const int lst = dz ? 0 : 16 * TL * 16;  // limb 1's image
      const int* eb = dz ? reinterpret_cast<const int*>(lds) : reinterpret_cast<const int*>(meta) + g * tlr + m_tok;
      // per (tile, limb) one chain of four MFMAs from zero; k-step j's B operand is formed once and feeds both limbs'
      // chains of every tile.  Every partial sum is an integer below 2^21 (|limb| <= 2048, |q| <= 8, 128 inputs), so
      // the sums are exact
      f32x4 D[NTT][2];
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) D[tt][0] = D[tt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f16x8 B = mm_b<BITS>(b0, b1, j);
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
          for (int l = 0; l < 2; ++l) {
            f16x8 A;
            __builtin_memcpy(&A, ab + (size_t)l * lst + (size_t)j * jst + tt * 256, 16);
            D[tt][l] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, D[tt][l], 0, 0, 0);
          }
      }
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) {
        const f32x4 dh = D[tt][0], dl = D[tt][1];
        const i32x4 xe = *reinterpret_cast<const i32x4*>(eb + 16 * tt);  // activation scale per token
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // the group sum sum(x_int * q) rounded once to fp32 (hi * 2048 exact inside the fma), times scale * 2^(E-148)
          const float gsum = fmaf(dh[i], 2048.0f, dl[i]);
          acc[b][tt][s][i] = fmaf(gsum, sc[s] * __int_as_float(xe[i]), acc[b][tt][s][i]);
        }
      }
    }
    const int rq = q - qa;
    if (ok && ((rq < 64 ? ends0 >> rq : ends1 >> (rq - 64)) & 1ull) != 0) {
      const int ep = stripe_of(rq);
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int o = (bl * MP + 16 * tt + 4 * h + i) * 16 + c;
          // the stripe's partial: its four group slots added in order
          const float part = ((acc[b][tt][0][i] + acc[b][tt][1][i]) + acc[b][tt][2][i]) + acc[b][tt][3][i];
          if constexpr (SK) {
            reinterpret_cast<float*>(outl)[o] = part;
          } else {
            yrun[b][tt][i] = ep == 0 ? part : yrun[b][tt][i] + part;
            if (ep == P - 1) reinterpret_cast<uint16_t*>(outl)[o] = f2bf(yrun[b][tt][i]);
          }
#pragma unroll
          for (int sl = 0; sl < 4; ++sl) acc[b][tt][sl][i] = 0.f;
        }
    }
  };

  // waves without a block skip the item loops (they take part in the staging and its barriers only)
  const bool busy = wave < nb;
  QuadRaw<BITS> buf[2];
  if (busy) {
    fetch_next(buf[0]);
    fetch_next(buf[1]);
  }
  // the item pairs of one (round, chunk): both items, then their stripe ends (LDS only), so that every load stays
  // outside any branch
  auto items = [&](int rd, int ch) __attribute__((always_inline)) {
    if (wave + NWV * NBW * rd >= nb) return;  // no block of this wave in this round (nor in any later one)
    const int q0 = qa + ch * cq, nq = qb - q0 < cq ? qb - q0 : cq, nit = seg_items(ch);
    for (int i0 = 0; i0 < nit; i0 += U) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (u) asm volatile("" ::: "memory");  // one item's operands live at a time
        const int b = NBW == 1 ? 0 : u;
        const int qi = NBW == 1 ? i0 + u : i0 / NBW;
        const int bl = wave + NWV * (NBW * rd + b);
        const bool ok = qi < nq && bl < nb;
        if (b == 0)
          core(buf[u], std::integral_constant<int, 0>(), q0 + (qi < nq ? qi : 0), q0, ok, bl);
        else
          core(buf[u], std::integral_constant<int, NBW - 1>(), q0 + (qi < nq ? qi : 0), q0, ok, bl);
        fetch_next(buf[u]);
      }
    }
  };
  if (tid < kZeros / 4) reinterpret_cast<uint32_t*>(lds)[tid] = 0u;
  if (nch == 1 && nrounds == 1) {  // the common case: one image, one round
    stage(0);
    __syncthreads();
    if (busy) items(0, 0);
  } else {
    for (int rd = 0; rd < nrounds; ++rd) {
      for (int ch = 0; ch < nch; ++ch) {
        if (nch > 1 || rd == 0) {
          if (rd + ch > 0) __syncthreads();  // every wave is done with the previous image
          stage(ch);
          __syncthreads();
        }
        if (busy) items(rd, ch);
      }
    }
  }

  __syncthreads();
  if constexpr (!SK) {
    for (int i = tid; i < nb * MP * 16; i += blockDim.x) {
      const int bl = i / (MP * 16), o = i - bl * MP * 16, t = o >> 4, row = (b_lo + bl) * 16 + (o & 15);
      if (t < m && row < n) yseg[(size_t)t * ldy + row] = reinterpret_cast<const uint16_t*>(outl)[i];
    }
  } else {
    // the stripe partials to scratch, device-coherent; every store is acknowledged at device scope before the range's
    // counter moves; the range's last workgroup adds the P partials of each output in stripe order
    for (int i = tid; i < nb * MP * 16; i += blockDim.x) {
      const int bl = i / (MP * 16), o = i - bl * MP * 16, t = o >> 4;
      __hip_atomic_store(spart + (((size_t)psk * n_b16 + b_lo + bl) * MP + t) * 16 + (o & 15),
                         reinterpret_cast<const float*>(outl)[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    int* const last = reinterpret_cast<int*>(lds);
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(scnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last = old == P - 1;
      if (old == P - 1) __hip_atomic_store(scnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
    }
    __syncthreads();
    if (!*last) return;
    // two outputs per thread at a time (block-major partials: the workgroup's outputs are the contiguous run from
    // b_lo * MP * 16); padding tokens and rows past n are summed and not written
    const int ne = nb * MP * 16, st = blockDim.x;
    for (int i0 = tid; i0 < ne; i0 += 2 * st) {
      const size_t off[2] = {(size_t)b_lo * MP * 16 + i0, (size_t)b_lo * MP * 16 + (i0 + st < ne ? i0 + st : i0)};
      float y[2];
      sum_stripe_partials_n<2>(spart, off, (size_t)MP * n_b16 * 16, P, y);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = i0 + u * st;
        const int bl = i / (MP * 16), o = i - bl * MP * 16, t = o >> 4, row = (b_lo + bl) * 16 + (o & 15);
        if (i < ne && t < m && row < n) yseg[(size_t)t * ldy + row] = f2bf(y[u]);
      }
    }
  }
}

template <int BITS, int NTT, int NBW, bool SK>
void launch_mm_k(const MmArgs& a, int grid, size_t smem, hipStream_t s) {
  const dim3 blk(mm_waves<NTT>() * 64);
  if constexpr (NTT == 1) {
    if (a.tl == 4)
      hipLaunchKernelGGL((mm_kernel<BITS, 1, NBW, SK, 4>), dim3(grid), blk, smem, s, a);
    else if (a.tl == 8)
      hipLaunchKernelGGL((mm_kernel<BITS, 1, NBW, SK, 8>), dim3(grid), blk, smem, s, a);
    else
      hipLaunchKernelGGL((mm_kernel<BITS, 1, NBW, SK, 16>), dim3(grid), blk, smem, s, a);
  } else {
    hipLaunchKernelGGL((mm_kernel<BITS, NTT, NBW, SK, 16 * NTT>), dim3(grid), blk, smem, s, a);
  }
}

// one or two blocks per wave and round (more would spill: rounds instead), for nb blocks per workgroup
template <int BITS, int NTT, bool SK>
void launch_nbw(const MmArgs& a, int nb, int grid, size_t smem, hipStream_t s) {
  if (nb > mm_waves<NTT>()) return launch_mm_k<BITS, NTT, 2, SK>(a, grid, smem, s);
  launch_mm_k<BITS, NTT, 1, SK>(a, grid, smem, s);
}

// image bytes of cq quads at token stride tl
size_t mm_image_bytes(int cq, int tl) { return kZeros + (size_t)cq * 4 * (2 * 16 * tl * 16 + tl * 4); }

template <int BITS, int NTT>
int launch_mm(MmArgs a, hipStream_t s) {
  const Segs& g = a.segs;
  const int ntile = a.nquad / 2;
  for (int i = 0; i < g.nseg; ++i)  // buffer offsets are 32-bit
    if ((long long)ntile * g.n[i] * 128 * BITS >= (1ll << 31)) return AK_INVALID;
  if ((long long)a.m * a.k * (a.act ? 4 : 2) >= (1ll << 31)) return AK_INVALID;
  int total = 0;
  for (int i = 0; i < g.nseg; ++i) total += (g.n[i] + 15) / 16;
  const int cus = num_cus();
  const size_t quad_bytes = mm_image_bytes(1, a.tl) - kZeros;

  // split-K across workgroups where the launch has few rows per CU (two 16-row blocks per CU or fewer): row ranges
  // shared out over the segments by their blocks, P workgroups per range, one stripe each
  // (more row ranges than CUs / P where a range's partials would leave too little LDS for the image: rounds of
  // workgroups)
  for (int f = 1; a.P >= 2 && total <= 2 * cus && f <= 4; f *= 2) {
    const int nrt = cus / a.P * f;
    if (nrt * a.P > 1024 || nrt < g.nseg) break;
    int nr[kMaxSegs] = {0, 0, 0, 0}, left = nrt - g.nseg;
    size_t part_floats = 0;
    for (int i = 0; i < g.nseg; ++i) {
      const int nbs = (g.n[i] + 15) / 16;
      nr[i] = 1 + (int)((long long)(left > 0 ? left : 0) * nbs / total);
      part_floats += (size_t)a.P * 16 * NTT * nbs * 16;
    }
    int sq = 0;  // quads of the widest stripe
    for (int p = 0; p < a.P; ++p) {
      const int w = stripe_begin(p + 1, a.nquad, a.P, 2) - stripe_begin(p, a.nquad, a.P, 2);
      sq = w > sq ? w : sq;
    }
    int nbr = 0;  // blocks of the widest row range
    for (int i = 0; i < g.nseg; ++i) {
      const int nbs = (g.n[i] + 15) / 16;
      nbr = (nbs + nr[i] - 1) / nr[i] > nbr ? (nbs + nr[i] - 1) / nr[i] : nbr;
    }
    const size_t outb = (size_t)nbr * 16 * NTT * 16 * 4;
    const int cq_max = outb + kZeros < kLds ? (int)((kLds - outb - kZeros) / quad_bytes) : 0;
    if (cq_max < 2) continue;  // a chunk holds at least two quads
    void* z = stream_scratch(s, 4096 + part_floats * 4);
    if (!z) break;
    MmArgs b = a;
    for (int i = 0, e = 0; i < kMaxSegs; ++i) {
      if (i < g.nseg) e += nr[i] * a.P;
      b.wg_end[i] = e;
    }
    b.cnt = static_cast<int*>(z);
    b.part = reinterpret_cast<float*>(static_cast<uint8_t*>(z) + 4096);
    const int cq2 = cq_max & ~1;  // a stripe has an even number of quads: chunks of an even number
    const int nch = (sq + cq2 - 1) / cq2;
    b.cq = ((sq + nch - 1) / nch + 1) & ~1;
    launch_nbw<BITS, NTT, true>(b, nbr, b.wg_end[g.nseg - 1], mm_image_bytes(b.cq, a.tl) + outb, s);
    return (int)hipGetLastError();
  }
  // one workgroup per CU, about the same number of blocks each, every workgroup within one segment
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
    const int nbs = (g.n[i] + 15) / 16, gsn = (nbs + per - 1) / per;
    nbmax = (nbs + gsn - 1) / gsn > nbmax ? (nbs + gsn - 1) / gsn : nbmax;
  }
  const size_t outb = (size_t)nbmax * 16 * NTT * 16 * 2;
  const int cq_max = outb + kZeros < kLds ? (int)((kLds - outb - kZeros) / quad_bytes) : 0;
  if (cq_max < 1) return AK_INVALID;
  // chunks of an even number of quads (nquad is even): with one block per wave the items come in pairs
  const int cq2 = cq_max & ~1;
  if (cq2 < 2) return AK_INVALID;
  const int nch = (a.nquad + cq2 - 1) / cq2;
  a.cq = ((a.nquad + nch - 1) / nch + 1) & ~1;
  launch_nbw<BITS, NTT, false>(a, nbmax, grid, mm_image_bytes(a.cq, a.tl) + outb, s);
  return (int)hipGetLastError();
}

}  // namespace

// 1..128 tokens in launches of at most 32 (one or two 16-token tiles per launch), group 128; act = 1: x is the merged
// gate_up [m][2k] and the activations SiLU(gate) * up.  AK_INVALID if the shape does not suit the kernel (the caller
// falls back).
int mm_gemv(int bits, const void* x, int m, const Segs& g, int k, int group, hipStream_t s, int act) {
  if (group != kG || m < 1 || m > 128 || bits < 2 || bits > 4) return AK_INVALID;
  for (int m0 = 0; m0 < m; m0 += kMaxTok) {
    const int mm = m - m0 < kMaxTok ? m - m0 : kMaxTok;
    MmArgs a;
    a.segs = g;
    for (int i = 0; i < g.nseg; ++i) a.segs.y[i] = g.y[i] + (size_t)m0 * g.ldy[i];
    a.x = static_cast<const uint16_t*>(x) + (size_t)m0 * (act ? 2 * (size_t)k : (size_t)k);
    a.act = act;
    a.m = mm;
    a.k = k;
    a.nquad = kpad(k) / kG / 4;
    a.P = stripe_count(a.nquad, 2);
    const int ntt = mm <= 16 ? 1 : 2;
    a.tl = ntt == 1 ? (mm <= 4 ? 4 : mm <= 8 ? 8 : 16) : 16 * ntt;
    a.cq = 1;
    a.part = nullptr;
    a.cnt = nullptr;
    for (int i = 0; i < kMaxSegs; ++i) a.wg_end[i] = 0;
    int e;
    switch (bits * 10 + ntt) {
      case 41: e = launch_mm<4, 1>(a, s); break;
      case 31: e = launch_mm<3, 1>(a, s); break;
      case 21: e = launch_mm<2, 1>(a, s); break;
      case 42: e = launch_mm<4, 2>(a, s); break;
      case 32: e = launch_mm<3, 2>(a, s); break;
      default: e = launch_mm<2, 2>(a, s); break;
    }
    if (e) return e;
  }
  return 0;
}

}  // namespace agq
