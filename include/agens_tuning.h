/* libagens_kernels: tuning entry points of the one- and two-token GEMV (the role of the reference's tuning entries,
 * kernels/include/agens_kernels.h:271-277 ak_w4g128_gemv_kt_tune / _variant and the launch pins of
 * tools/aot_pins_sm90.json, produced by kernels/bench/tune_w4.cu:1-91).  Every launch configuration gives the same
 * output bits; these only select among them.  Used by agens-engine_amd/tune_launch.py, which measures the candidates
 * and writes the compiled-in table (csrc/wq_launch_table.h) that ak_wq_gemv_kt_multi consults.  Not for engines:
 * every switch here is process-global (it changes the launches of every thread until it is reset) and meant for
 * tuning and tests. */
#pragma once

#ifdef __cplusplus
extern "C" {
#endif

/* Forces the launch configuration of the following one- and two-token GEMV launches (group 128, default numerics) in
 * this process: split = stripe sets per 4-row block (1, 2, 4, 8; 0: not forced), nwv = waves per workgroup (16, 8;
 * 0: not forced), sk = split-K across workgroups (1 yes, 0 no, -1 not forced, -2 not forced and the measured pins
 * ignored: the cost model alone).  A forced value the shape does not admit is ignored for that launch.  Always 0. */
int ak_wq_tune_override(int split, int nwv, int sk);

/* The configuration a one- or two-token launch (m = 1, 2) of these segments takes now (pins, override and cost model
 * applied): 0 and *split, *nwv, *sk (1: split-K across workgroups), or 1 if the shape is not one this kernel takes. */
int ak_wq_tune_query(int bits, int m, int nseg, const int* n, int k, int* split, int* nwv, int* sk);

/* The smallest token count (m) that ak_wq_gemv_kt_multi and its conveniences route to the fp16-MFMA kernel in the
 * default numerics (group 128): m >= this many tokens take it, fewer take the integer-limb kernels, at every k.  0:
 * never (the integer-limb kernels for every m); negative: the compiled-in measured rule (17 tokens and k <= 8192; or
 * the environment variable AGENS_WQ_MM_MIN).  Both kernels compute the same numerics bit for bit, so this changes
 * speed only.  Process-wide.  Always 0. */
int ak_wq_set_mm_min(int m);

#ifdef __cplusplus
}
#endif
