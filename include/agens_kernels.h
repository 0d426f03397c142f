/* libagens_kernels (MI355X / gfx950 build): the C ABI of the mixed-bit group-quantized linear-layer path.
 *
 * Drop-in for the quantized-GEMV part of the reference's kernels/include/agens_kernels.h: same names, argument order,
 * argument meaning and return codes, so crates/agens-cuda/src/lib.rs:9-35 (Rust FFI) and the model's linear()
 * (kernels/m1/m1_model.cu:1857-1937) bind to it unchanged.  Each declaration cites the reference declaration it
 * replaces.  Entry points of the reference header that are not part of this path are not exported.
 *
 * Conventions (reference header :1-2):
 *   - every int-returning function returns 0 on success or an error code with the reference's numeric meaning:
 *     1 = invalid value (bad shape / group, or a value that needs more bits than requested), 2 = out of memory,
 *     other values are hipError_t codes;
 *   - `stream` is a hipStream_t (NULL = the default stream); launches are asynchronous and stream-ordered;
 *   - bf16 tensors are passed as void* (raw 16-bit patterns), the int4 container as int32_t words;
 *   - the caller owns every buffer it passes.  The GEMV entry points (and ak_wq_gemm_kt on narrow linears) own scratch
 *     only for split-K launches (long k, or few rows per CU, at more than two tokens or long k): per (device, stream),
 *     allocated zero-filled on the first such call outside a stream capture (that call synchronizes the device once),
 *     grown (at least doubling) when a larger launch needs it; every buffer, a replaced one included, is held until
 *     the process ends -- as the reference's split-K scratch (w4_gemv.cu:2096-2118) -- so graphs captured before a
 *     growth stay valid.  Inside a capture they never allocate or synchronize: without scratch they take a launch
 *     that needs none (the GEMV: same results; the GEMM: k not split), so they can be captured in a hipGraph.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------------- runtime
 * reference: kernels/include/agens_kernels.h:17-30 (implemented in kernels/src/runtime.cu:25-44). */
int ak_device_count(int* n);                                  /* agens_kernels.h:17 */
int ak_set_device(int dev);                                   /* agens_kernels.h:18 */
int ak_device_name(int dev, char* buf, int len);              /* agens_kernels.h:19 */
int ak_malloc(void** ptr, size_t bytes);                      /* agens_kernels.h:20 */
int ak_free(void* ptr);                                       /* agens_kernels.h:21 */
int ak_memcpy_h2d(void* dst, const void* src, size_t bytes);  /* agens_kernels.h:22 */
int ak_memcpy_d2h(void* dst, const void* src, size_t bytes);  /* agens_kernels.h:23 */
int ak_synchronize(void);                                     /* agens_kernels.h:24 */
int ak_mem_info(size_t* free_bytes, size_t* total_bytes);     /* agens_kernels.h:25 */
const char* ak_error_string(int code);                        /* agens_kernels.h:28 */
int ak_host_alloc(void** ptr, size_t bytes);                  /* agens_kernels.h:29: pinned host memory */
int ak_host_free(void* ptr);                                  /* agens_kernels.h:30 */

/* ---------------------------------------------------------------------------------------------- sizes
 * KT ("k-tiled") layout: k padded to kp = ceil(k / 1024) * 1024; tile t of row o is one record at
 * (t * n + o) * (128 * bits) bytes; scales bf16 at (t * n + o) * (1024 / group).  reference: w4_gemv.cu:13-31. */
size_t ak_w4_kt_weight_bytes(int n, int k);               /* agens_kernels.h:192, w4_gemv.cu:560 */
size_t ak_w4_kt_scale_bytes(int n, int k, int group);     /* agens_kernels.h:193, w4_gemv.cu:561 */
size_t ak_w3_kt_weight_bytes(int n, int k);               /* agens_kernels.h:240, w4_gemv.cu:822 */
size_t ak_wq_kt_weight_bytes(int bits, int n, int k);     /* agens_kernels.h:255, w4_gemv.cu:821 */
size_t ak_w4g128_kt_weight_bytes(int n, int k);           /* agens_kernels.h:181, w4_gemv.cu:562 */
size_t ak_w4g128_kt_scale_bytes(int n, int k);            /* agens_kernels.h:182, w4_gemv.cu:563 */

/* ---------------------------------------------------------------------------------------------- load-time repack
 * int4 container (packed int32 [n][k/8], nibble = q + 8, low nibble first; scales bf16 [n][k/group]) -> KT.
 * group in {64, 128}, k % group == 0, k % 32 == 0, else 1.  W3 / W2: 1 if a value needs more bits (the layout is
 * written anyway; the caller keeps the linear wider).  The W3 / W2 entry points synchronize the stream. */
int ak_w4_repack_kt(const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, int group,
                    void* stream);                        /* agens_kernels.h:194, w4_gemv.cu:565-583 */
int ak_w3_repack_kt(const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, int group,
                    void* stream);                        /* agens_kernels.h:241, w4_gemv.cu:845-848 */
int ak_wq_repack_kt(int bits, const int32_t* packed, const void* scales, void* wt, void* st, int n, int k, int group,
                    void* stream);                        /* agens_kernels.h:256-257, w4_gemv.cu:826-844 */
int ak_w4g128_repack_kt(const int32_t* packed, const void* scales, void* wt, void* st, int n, int k,
                        void* stream);                    /* agens_kernels.h:183, w4_gemv.cu:585-588 */

/* ---------------------------------------------------------------------------------------------- GEMV / small-M GEMM
 * x bf16 [m][k] (rows contiguous, stride k, 16-byte aligned); y bf16, token j of segment i at y[i] + j * ldy[i]
 * (ldy == NULL: n[i]).  1 <= m <= 128, 1 <= nseg <= 4, the segments share x, k, group and bits.
 * Numerics (both deterministic; every output row is bit-identical for any m, any segmentation and any bit width
 * holding the same values):
 *   default  -- integer MFMA: per group of inputs, x as fixed point relative to the group's largest input,
 *               x_int = trunc(x * 2^(148 - E)) with E that input's exponent field (22 bits: inputs below 2^-14 of the
 *               group's largest lose their low bits), the integer dot product of q with x_int exact, rounded once
 *               to fp32, scaled and accumulated in fp32 in a fixed order.  Non-finite inputs: a group holding a NaN
 *               adds NaN; one holding an Inf (no NaN) adds S * scale * Inf, S the sum of sign(x) * q over its Infs
 *               (+-Inf, or NaN where S = 0: the fp32 path's value wherever the group's Inf products share a sign).
 *               Groups whose largest input is below about 2^-100 lose precision to the underflow of the fp32 scale
 *               product (absolute errors below 2^-100), where the reference's fp32 per-group path
 *               (reference.rs:53-71) keeps them;
 *   exact    -- the reference's fp32 FMA path, bit for bit (ak_w4_set_mma(0) or AGENS_W4_EXACT=1);
 *   bf16w=1  -- weights rounded to bf16(q * scale) first (Marlin numerics), always on the fp32 path. */
int ak_wq_gemv_kt_multi(int bits, const void* x, int m, int nseg, const void* const* wt, const void* const* st,
                        void* const* y, const int* n, const int* ldy, int k, int group, int bf16w,
                        void* stream);            /* agens_kernels.h:258-259, w4_gemv.cu:852-876 */
/* No counterpart in the reference: ak_wq_gemv_kt_multi that allocates nothing, for callers that cannot call hipMalloc
 * (code under stream capture, tight serving loops, harnesses that forbid allocation).  Same arguments, results and
 * error codes; its split-K launches keep their partials and counters in a static 64 MiB device array of the library
 * (one per GPU, held until the process ends) instead of per-stream scratch.  Returns 1 when the call's worst-case
 * scratch on its route, 4096 + 64 * P * T * sum_i ceil(n[i] / 16) bytes (P = min(8, ceil(k / 1024)); T = 4, 8 or 16
 * for up to 4, 8 or 16 tokens on the integer kernels, 16 or 32 for up to 16 or more tokens on the fp16-MFMA route that
 * the default numerics take from 17 tokens at k <= 8192), exceeds it (e.g. a 152064-row linear at more than 8 tokens).
 * Calls that overlap in time on one GPU share the array and race: keep them on one stream. */
int ak_wq_gemv_kt_multi_noalloc(int bits, const void* x, int m, int nseg, const void* const* wt,
                                const void* const* st, void* const* y, const int* n, const int* ldy, int k, int group,
                                int bf16w, void* stream);
int ak_w4_gemv_kt(const void* x, const void* wt, const void* st, void* y, int n, int k, int group, int bf16w,
                  void* stream);                  /* agens_kernels.h:195-196, w4_gemv.cu:702-710 */
int ak_w4_gemv_kt_multi(const void* x, int nseg, const void* const* wt, const void* const* st, void* const* y,
                        const int* n, int k, int group, int bf16w, void* stream); /* agens_kernels.h:197-198, w4_gemv.cu:712-720 */
int ak_w4_gemv_kt_batched(const void* x, const void* wt, const void* st, void* y, int m, int n, int k, int group,
                          int bf16w, void* stream); /* agens_kernels.h:199-200, w4_gemv.cu:722-731 */
int ak_w3_gemv_kt(const void* x, const void* wt, const void* st, void* y, int n, int k, int group,
                  void* stream);                  /* agens_kernels.h:242 */
int ak_w3_gemv_kt_multi(const void* x, int nseg, const void* const* wt, const void* const* st, void* const* y,
                        const int* n, int k, int group, void* stream); /* agens_kernels.h:243-244 */
int ak_w3_gemv_kt_batched(const void* x, const void* wt, const void* st, void* y, int m, int n, int k, int group,
                          void* stream);          /* agens_kernels.h:245-246 */
/* reference: the tensor-core entry point (agens_kernels.h:204, w4_gemv.cu:3265-3270); here: the default numerics */
int ak_w4_mma_gemv(const void* x, const void* wt, const void* st, void* y, int m, int n, int k, int group,
                   void* stream);
/* g128 conveniences (agens_kernels.h:184, :48-49): KT and the legacy int4-container (CT) GEMV, exact numerics */
int ak_w4g128_gemv_kt_bf16(const void* x, const void* wt, const void* st, void* y, int n, int k, void* stream);
int ak_w4g128_gemv_bf16(const void* x, const int32_t* packed, const void* scales, void* y, int n, int k,
                        void* stream);
/* tuning entries (agens_kernels.h:271-277, w4_gemv.cu:590-651, :916-935): every variant returns the same bits */
int ak_w4g128_gemv_bf16_variant(int variant, const void* x, const int32_t* packed, const void* scales, void* y,
                                int n, int k, void* stream);
int ak_w4g128_gemv_kt_variant(int variant, const void* x, const void* wt, const void* st, void* y, int n, int k,
                              void* stream);
int ak_w4g128_gemv_kt_tune(int r, int u, int warps, int bps, const void* x, const void* wt, const void* st, void* y,
                           int n, int k, void* stream);

/* ---------------------------------------------------------------------------------------------- dequant (prefill)
 * rows [r0, r0 + nr) -> w bf16 [nr][k], value bf16_rn(q * scale), bitwise.  reference: w4_gemv.cu:460-493. */
int ak_wq_dequant_kt_rows(int bits, const void* wt, const void* st, void* w, int n, int k, int group, int r0, int nr,
                          void* stream);          /* agens_kernels.h:260-261, w4_gemv.cu:877-895 */
int ak_w4_dequant_kt(const void* wt, const void* st, void* w, int n, int k, int group,
                     void* stream);               /* agens_kernels.h:265, w4_gemv.cu:733-741 */
int ak_w4_dequant_kt_rows(const void* wt, const void* st, void* w, int n, int k, int group, int r0, int nr,
                          void* stream);          /* agens_kernels.h:267-268, w4_gemv.cu:743-752 */
int ak_w3_dequant_kt_rows(const void* wt, const void* st, void* w, int n, int k, int group, int r0, int nr,
                          void* stream);          /* agens_kernels.h:247-248 */

/* ---------------------------------------------------------------------------------------------- prefill GEMM
 * y[m][ldy] = x[m][k] W^T, bf16 x and W [n][k] (the dequantized rows of ak_wq_dequant_kt_rows), fp32 accumulation,
 * bf16 y; the model's linear() takes this route above 128 tokens.  A library GEMM (rocBLAS gemm_ex), not a kernel of
 * this library; its accumulation order is the library's (results within fp32-accumulation tolerance of the oracle). */
int ak_bf16_linear_f32reduce(const void* x, const void* w, void* y, int m, int n, int k,
                             void* stream);       /* agens_kernels.h:55, bf16_linear.cu:82-92 */
int ak_bf16_linear_f32reduce_ld(const void* x, const void* w, void* y, int m, int n, int k, int ldy,
                                void* stream);    /* agens_kernels.h:56, bf16_linear.cu:68-80 */

/* ---------------------------------------------------------------------------------------------- fused prefill GEMM
 * No single counterpart in the reference: ak_wq_dequant_kt_rows followed by ak_bf16_linear_f32reduce_ld in one kernel,
 * the pair the model's linear() runs above 128 tokens (kernels/m1/m1_model.cu:1876-1897, w4_gemv.cu:877-895,
 * bf16_linear.cu:68-80).  y[t][o] (row stride ldy; 0: n) = bf16(sum_i x[t][i] * w[o][i]) for every token t < m and
 * row o < n of a KT linear, w[o][i] = bf16_rn(q * scale) (the dequantized values, bit for bit), fp32 accumulation in
 * this kernel's order (within fp32-accumulation error of the two-call route); no weight copy.  Where the linear has
 * few output tiles (fewer than 384 of 128 rows x 128 tokens) k is split across workgroups: fp32 partials in the
 * stream's split-K scratch (above), added in a fixed order by a second kernel, so results are deterministic for a
 * given shape.  group in {64, 128}, k % group == 0, ldy >= n, else 1. */
int ak_wq_gemm_kt(int bits, const void* x, int m, const void* wt, const void* st, void* y, int n, int ldy, int k,
                  int group, void* stream);

/* ---------------------------------------------------------------------------------------------- INT8 LM head GEMV
 * W8A16: y[j][o] (row stride ldy) = bf16(scale[o] * sum_i x[j][i] * q[o][i]); q int8 [n][k] row-major, scale fp32 [n]
 * (per-row symmetric), x bf16 [m][k]; 1 <= m <= 16, k % 16 == 0 (else 1).  The reference's fp32 order (32 chunk-strided
 * partials of 16-input fma chains, xor butterfly), kept exactly: bit-identical to the reference, and row j of an
 * m-token call is bit-identical to the 1-token call. */
int ak_i8_gemv(const void* x, const void* w, const void* scale, void* y, int m, int n, int k, int ldy,
               void* stream);                     /* agens_kernels.h:264, i8_gemv.cu:72-88 */

/* ---------------------------------------------------------------------------------------------- batch-invariant bf16 GEMV
 * y[t][r] (row stride ldy; n for ak_bf16_gemv_bi) = bf16(sum_i x[t][i] W[r][i] (+ bias[r])); W bf16 [n][k] row-major,
 * x bf16 [m][k], bias bf16 [n] or NULL; 1 <= m <= 128, k % 32 == 0 (else 1).  fp32 accumulation (MFMA), the bias added
 * in fp32 before the one bf16 rounding, and a summation order that does not depend on m: row t of an m-token call is
 * bit-identical to the 1-token call.  The reference's bits come from its tensor-core MMA's internal accumulation, so
 * results agree with the reference within fp32-accumulation tolerance, not bit for bit. */
int ak_bf16_gemv_bi(const void* x, const void* w, const void* bias, void* y, int m, int n, int k,
                    void* stream);                /* agens_kernels.h:88, bi_gemv.cu:270-273 */
int ak_bf16_gemv_bi_ld(const void* x, const void* w, const void* bias, void* y, int m, int n, int k, long ldy,
                       void* stream);             /* agens_kernels.h:89, bi_gemv.cu:274-356 */

/* ---------------------------------------------------------------------------------------------- SiLU(gate) * up
 * out[t][i] = bf16(g / (1 + exp(-g)) * u) for g = gate_up[t][i], u = gate_up[t][inter + i] (the merged gate_up output
 * [tokens][2 inter] -> [tokens][inter]); inter % 8 == 0 (else 1).  _part: one tensor-parallel share [gate share | up
 * share] (np each) -> the full row of inter, the share's products at [lo, lo + np) and zeros elsewhere.  The
 * reference compiles the expression with CUDA's fast-math exp and division; here exp is the device library's expf and
 * the division an fp32 division: results within one bf16 unit in the last place of the reference's, not bit for bit. */
int ak_silu_mul(const void* gate_up, void* out, int tokens, int inter,
                void* stream);                    /* agens_kernels.h:110, silu_mul.cu:66-72 */
int ak_silu_mul_part(const void* gate_up_part, void* out, int inter, int lo, int np,
                     void* stream);               /* agens_kernels.h:113, silu_mul.cu:58-64 */

/* ---------------------------------------------------------------------------------------------- fused SiLU(gate) * up
 * No counterpart in the reference: ak_silu_mul followed by ak_wq_gemv_kt_multi in one launch, for the down projection
 * of a decoder layer (the reference runs the two, kernels/m1/m1_model.cu:2583).  y[t] (row stride ldy; 0: n) =
 * W . act[t], act[t][i] = bf16(SiLU(gate_up[t][i]) * gate_up[t][inter + i]) (ak_silu_mul's value, bit for bit),
 * gate_up bf16 [m][2 inter]; W the KT layout of an n x inter linear.  Results are bit-identical to ak_silu_mul
 * followed by ak_wq_gemv_kt_multi.  The default numerics at group 128 only: otherwise (group 64, the exact path)
 * it returns 1 and the caller runs the two calls. */
int ak_wq_gemv_kt_silu(int bits, const void* gate_up, int m, const void* wt, const void* st, void* y, int n, int ldy,
                       int inter, int group, void* stream);

/* ---------------------------------------------------------------------------------------------- chained GEMV steps
 * No single counterpart in the reference: it replaces a run of ak_wq_gemv_kt_multi launches joined by programmatic
 * dependent launch edges in a captured graph (reference: ak_graph_pdl, kernels/src/runtime.cu:198-230, and the
 * kernel-side contract of kernels/include/agens_pdl.cuh:1-16: a GEMV may read its constant weights before the kernel
 * it depends on has finished, and reads x / writes y only after).  MI355X has no programmatic launch edges between
 * same-stream kernels, so the steps run in ONE persistent launch: each step issues its first weight loads, waits for
 * every workgroup to finish the previous step (a grid barrier over per-workgroup flag words in device memory), then
 * reads its activations.  Results are bit-identical to running the steps one ak_wq_gemv_kt_multi call each, in order.
 *
 * A step has ak_wq_gemv_kt_multi's arguments (ldy[i] = 0: n[i]).  independent = 1 declares that the step reads and
 * writes nothing that the steps since the last dependent step write (or read, for its writes): it then does not wait.
 * The chained kernels take steps of group 128 on the default numerics: with m <= 2 the line-load kernel's steps, with
 * m <= 4 (no act step) the tokens-in-A-rows kernel's; any other chain runs as one ak_wq_gemv_kt_multi call per step
 * (same results, no overlap).
 *   ak_wq_chain_create  validates the steps (as ak_wq_gemv_kt_multi: 1 on a bad argument), allocates and uploads the
 *                       chain's step table (device memory, synchronous); not under stream capture;
 *   ak_wq_chain_run     one launch on `stream`, allocates nothing, capturable; at most one chained launch may run on
 *                       a device at a time (they share the device's flag words): outside capture, a launch on another
 *                       stream than the device's last chained launch is refused with 600 (hipErrorNotReady) while that
 *                       launch has not finished;
 *   ak_wq_chain_status  after the stream is synchronized: 1 if a chained launch's bounded wait (0.2 s) ran out since
 *                       the last call (its outputs are then not valid), else 0; negative: a HIP error. */
typedef struct ak_wq_step {
  int bits, m, nseg, k, group, bf16w;
  const void* x;
  const void* wt[4];
  const void* st[4];
  void* y[4];
  int n[4];
  int ldy[4];
  int independent;
  int act; /* 1: x is the merged gate_up [m][2k] and the step's activations are SiLU(gate) * up (ak_wq_gemv_kt_silu) */
} ak_wq_step;
int ak_wq_chain_create(const ak_wq_step* steps, int nsteps, void** chain);
int ak_wq_chain_run(void* chain, void* stream);
int ak_wq_chain_chained(void* chain); /* 1: runs as one chained launch, 0: one launch per step */
int ak_wq_chain_destroy(void* chain);
int ak_wq_chain_status(void);

/* ---------------------------------------------------------------------------------------------- switches
 * reference: agens_kernels.h:205 / :208 / :211, w4_gemv.cu:3271-3282.  mma: -1 auto (environment AGENS_W4_EXACT), 0 exact
 * fp32 path, 1 default integer-MFMA path.  lean / tma select bit-identical sm90-only variants in the reference;
 * accepted and ignored here (one kernel family per numerics). */
int ak_w4_set_mma(int mode);
int ak_w4_set_lean(int rb);
int ak_w4_set_tma(int stages);

#ifdef __cplusplus
}
#endif
