/* CPU oracle for the mixed-bit (W2/W3/W4) group-quantized GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or, for the CPU baseline, as the timed restatement of the reference's CPU path).
 * The product library (agens-engine_amd/) never links or calls it.
 *
 * Every function restates an algorithm of the reference (BlockWayz/agens-engine) and cites the file:line it follows.
 * bf16 values are passed as raw uint16_t bit patterns, the int4 container as uint32_t words.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 <-> fp32 (round to nearest even), as kernels/bench/test_w4.cu:41-51 */
float ora_bf2f(uint16_t b);
uint16_t ora_f2bf(float f);

/* ---- int4 container ("CT"): crates/agens-core/src/reference.rs:20-36 (pack_row / unpack_row) */
int ora_pack_row(const int8_t* q, int k, uint32_t* out);   /* returns -1 if a value is outside [-8, 7] */
void ora_unpack_row(const uint32_t* p, int k, int8_t* q);
/* reference.rs:38-51 quantize_row (group 128, round half away from zero, clamp [-8, 7]) */
void ora_quantize_row(const float* w, int k, int8_t* q, uint16_t* s);

/* ---- KT ("k-tiled") layouts: kernels/src/w4_gemv.cu:13-31 (spec), :439-458 (W4 repack), :756-790 (W3/W2 repack),
 * :560-563 / :821-822 (sizes), :565-583 / :826-844 (argument rules).  Return 0, or 1 (= invalid value: bad group / k,
 * or a value that needs more than `bits` bits; the layout is still written, as the reference's kernel does). */
size_t ora_kt_weight_bytes(int bits, int n, int k);
size_t ora_kt_scale_bytes(int n, int k, int group);
int ora_repack_kt(int bits, const uint32_t* packed, const uint16_t* scales, uint8_t* wt, uint16_t* st, int n, int k,
                  int group);
/* w4_gemv.cu:78-110 (ldw / spread2 / spread1 / w3_word / w2_word): lane chunk of record rec -> 4 W4 nibble words */
void ora_kt_chunk(int bits, const uint8_t* wt, size_t rec, int lane, uint32_t out[4]);
/* w4_gemv.cu:460-493 dequant_kt_kernel: rows [r0, r0+nr) -> w [nr][k] bf16, value bf16_rn(q * s) */
int ora_dequant_kt_rows(int bits, const uint8_t* wt, const uint16_t* st, uint16_t* w, int n, int k, int group, int r0,
                        int nr);

/* ---- adjacent GEMVs */
/* INT8 LM head (W8A16): kernels/src/i8_gemv.cu:28-70 (dot4, i8_gemv_kernel).  q int8 [n][k], scale fp32 [n], k % 16 == 0;
 * y[j * ldy + o] = bf16_rn(v * scale[o]), v = xor butterfly (distance 16, 8, 4, 2, 1: v[l] + v[l ^ d]) of 32 partials,
 * partial l = sum over the 16-input chunks c = l, l + 32, ... (in that order) of s, s = fmaf(x_e, q_e, s) from 0 over
 * the chunk's inputs e = 0..15. */
void ora_i8_gemv(const uint16_t* x, const int8_t* q, const float* scale, uint16_t* y, int m, int n, int k, int ldy);

/* ---- GEMV references.  x bf16 [m][k] (row stride k); y written per token j at y + j * ldy. */
/* reference.rs:53-71 (w4::gemv) generalised to group G: per group ga += x*q in fp32, then acc += ga * s (no fma).
 * Reads the int4 container.  nthreads > 1 splits output rows statically over POSIX threads (same bits). */
void ora_gemv_ref_f32(const uint16_t* x, int m, const uint32_t* packed, const uint16_t* scales, float* y, int ldy,
                      int n, int k, int group, int nthreads);
/* fp64 reference of the fp32-dequantised product and sum |x*w| (the bound of kernels/bench/test_w4.cu:123-141). */
void ora_gemv_ref_f64(const uint16_t* x, int m, const uint32_t* packed, const uint16_t* scales, double* y,
                      double* mag, int ldy, int n, int k, int group);
/* Bit-exact restatement of the reference's exact fp32 path on KT weights: w4_gemv_kt_kernel / _batched_kernel
 * (w4_gemv.cu:112-127 nib/dot8, :279-349, :367-437): lane l owns chunk 32t+l of every tile, per chunk a 32-input
 * fma chain, acc = fma(d, s, acc) (bf16w = 1: weights rounded to bf16(q*s), acc += d), xor butterfly 16..1, bf16 RN. */
void ora_gemv_exact_kt(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y,
                       int ldy, int n, int k, int group, int bf16w);
/* The default (integer-MFMA) numerics of this build, restated on the CPU:
 *  - per (token, group g): E = max bf16 exponent field of x over g; x_int = trunc(x * 2^(148-E)) (|x_int| < 2^22),
 *    balanced signed bytes x_int = d2 * 2^16 + d1 * 2^8 + d0; exact integer limb sums D_j = sum d_j * q;
 *    gsum = fmaf((float)(D2 * 256 + D1), 256, (float)D0) (= fp32_rn of the exact group dot product times 2^(148-E)
 *    unless |D2 * 256 + D1| >= 2^24); sE = scale * 2^(E-148) (fp32 multiply);
 *  - groups in quads of 4 (slot s = g % 4); the nt = kpad(k) / 1024 tiles in P = min(8, nt) contiguous stripes
 *    (stripe p = tiles [p * nt / P, (p + 1) * nt / P), i.e. whole tiles of quads);
 *    acc[p][s] = fmaf(gsum, sE, acc[p][s]) over the stripe's quads in order;
 *    part[p] = ((acc[p][0] + acc[p][1]) + acc[p][2]) + acc[p][3]; y = part[0] + part[1] + ... (left to right); bf16 RN.
 * Same semantics as reference.rs:53-71 (sum_g s_g * sum_{i in g} x_i q_i, fp32 accumulation); only the rounding
 * points differ (one rounding per group sum instead of one per product-add). */
void ora_gemv_fast_kt(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y, int ldy,
                      int n, int k, int group);
/* the same two GEMVs restricted to output rows [r0, r1) (y still indexed by the full row number) */
void ora_gemv_fast_kt_rows(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y,
                           int ldy, int n, int k, int group, int r0, int r1);
void ora_gemv_exact_kt_rows(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y,
                            int ldy, int n, int k, int group, int bf16w, int r0, int r1);
/* exact integer group sum of the fast numerics for one (token row x, weight row o, group g) -- exposes GS and E */
long long ora_fast_group_sum(int bits, const uint16_t* x, const uint8_t* wt, int n, int k, int group, int o, int g,
                             int* E);

/* ---- deterministic generators (reference test inputs) */
/* xorshift32 (kernels/bench/test_w4.cu:36-40, test_wq.cu:36-40) */
uint32_t ora_xorshift32(uint32_t* state);
/* counter-based generator for the BASELINE configs: uniform u32 of (seed, index) */
uint32_t ora_hash_u32(uint64_t seed, uint64_t index);
/* codes uniform in [lo, lo + span) written as container nibbles (q + 8); scales bf16(|N(0,1)|*sa + sb); x bf16(N(0,1)*xs) */
void ora_gen_container(uint64_t seed, int n, int k, int lo, int span, uint32_t* packed);
void ora_gen_scales(uint64_t seed, size_t count, float sa, float sb, uint16_t* s);
void ora_gen_x(uint64_t seed, size_t count, float xs, uint16_t* x);

#ifdef __cplusplus
}
#endif
