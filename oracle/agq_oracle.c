/* CPU oracle for the mixed-bit group-quantized GEMV path -- TEST INFRASTRUCTURE ONLY (see agq_oracle.h).
 *
 * Compiled with -ffp-contract=off: every a * b + c below is two roundings unless written as fmaf(), exactly as the
 * reference's Rust (reference.rs) and CUDA (w4_gemv.cu) code it restates.
 */
#include "agq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------ bf16 */
float ora_bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round to nearest even; kernels/bench/test_w4.cu:47-51 for finite values, NaN kept quiet */
uint16_t ora_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* ------------------------------------------------------------------------------------------------ container */
/* reference.rs:20-32: value q in [-8, 7] stored as nibble q + 8, 8 per word, lowest input in the lowest nibble */
int ora_pack_row(const int8_t* q, int k, uint32_t* out) {
  if (k % 8) return -1;
  for (int w = 0; w < k / 8; ++w) {
    uint32_t v = 0;
    for (int j = 0; j < 8; ++j) {
      const int x = q[8 * w + j];
      if (x < -8 || x > 7) return -1;
      v |= ((uint32_t)(x + 8) & 0xFu) << (4 * j);
    }
    out[w] = v;
  }
  return 0;
}

/* reference.rs:34-36 */
void ora_unpack_row(const uint32_t* p, int k, int8_t* q) {
  for (int i = 0; i < k; ++i) q[i] = (int8_t)((int)((p[i / 8] >> (4 * (i % 8))) & 0xFu) - 8);
}

/* reference.rs:38-51: symmetric per-group quantisation, group 128 */
void ora_quantize_row(const float* w, int k, int8_t* q, uint16_t* s) {
  for (int g = 0; g < k / 128; ++g) {
    const float* gw = w + 128 * g;
    float amax = 0.f;
    for (int i = 0; i < 128; ++i) amax = fmaxf(amax, fabsf(gw[i]));
    const uint16_t sb = ora_f2bf(amax == 0.f ? 1.f : amax / 7.f);
    const float sf = ora_bf2f(sb);
    for (int i = 0; i < 128; ++i) {
      float r = roundf(gw[i] / sf); /* Rust f32::round: half away from zero */
      if (r < -8.f) r = -8.f;
      if (r > 7.f) r = 7.f;
      q[128 * g + i] = (int8_t)r;
    }
    s[g] = sb;
  }
}

/* ------------------------------------------------------------------------------------------------ KT layouts */
static int kpad(int k) { return (k + 1023) & ~1023; }
static int group_ok(int k, int group) { return (group == 64 || group == 128) && k % group == 0; }

/* w4_gemv.cu:821 */
size_t ora_kt_weight_bytes(int bits, int n, int k) { return (size_t)n * kpad(k) * bits / 8; }
/* w4_gemv.cu:561 */
size_t ora_kt_scale_bytes(int n, int k, int group) { return (size_t)n * kpad(k) / group * 2; }

int ora_repack_kt(int bits, const uint32_t* packed, const uint16_t* scales, uint8_t* wt, uint16_t* st, int n, int k,
                  int group) {
  if ((bits < 2 || bits > 4) || !group_ok(k, group) || k % 32 != 0) return 1;
  const int SPT = 1024 / group, CPG = group / 32;
  const int tiles = kpad(k) >> 10, chunks = k >> 5, groups = k / group;
  const int OFF = 8 - (1 << (bits - 1)), MAXN = (1 << bits) - 1;
  int bad = 0;
  for (int t = 0; t < tiles; ++t)
    for (int o = 0; o < n; ++o) {
      const size_t rec = (size_t)t * n + o;
      for (int lane = 0; lane < 32; ++lane) {
        const int c = t * 32 + lane;
        uint32_t q[4];
        for (int i = 0; i < 4; ++i) q[i] = c < chunks ? packed[((size_t)o * chunks + c) * 4 + i] : 0x88888888u;
        if (bits == 4) {
          /* w4_gemv.cu:439-458: the 16-byte chunk is copied as is */
          memcpy(wt + (rec * 32 + lane) * 16, q, 16);
        } else {
          /* w4_gemv.cu:758-790: 2-bit low fields (inputs 0-15 word 2l, 16-31 word 2l+1, field at bit 2*(v&15)),
           * W3 third bit at word 64+l bit v; value n = nibble - OFF, range-checked */
          uint32_t lo[2] = {0u, 0u}, hi = 0u;
          for (int v = 0; v < 32; ++v) {
            const int nv = (int)((q[v >> 3] >> (4 * (v & 7))) & 0xFu) - OFF;
            if (nv < 0 || nv > MAXN) bad = 1;
            const uint32_t mv = (uint32_t)nv & (uint32_t)MAXN;
            lo[v >> 4] |= (mv & 3u) << (2 * (v & 15));
            if (bits == 3) hi |= (mv >> 2) << v;
          }
          uint32_t* b = (uint32_t*)wt + rec * (32 * bits);
          b[2 * lane] = lo[0];
          b[2 * lane + 1] = lo[1];
          if (bits == 3) b[64 + lane] = hi;
        }
        if (lane % CPG == 0) {
          const int g = c / CPG;
          st[rec * SPT + lane / CPG] = g < groups ? scales[(size_t)o * groups + g] : 0;
        }
      }
    }
  return bad;
}

/* w4_gemv.cu:78-110 (ldw): a W3 / W2 lane chunk read back as the W4 nibble words of the same values, written here
 * input by input from the layout definition (w4_gemv.cu:23-31): input v of the chunk has its 2-bit field in word
 * 2*lane + v/16 at bit 2*(v%16), and (W3) its third bit in word 64 + lane at bit v; nibble = n + (8 - 2^(bits-1)). */
void ora_kt_chunk(int bits, const uint8_t* wt, size_t rec, int lane, uint32_t out[4]) {
  if (bits == 4) {
    memcpy(out, wt + (rec * 32 + lane) * 16, 16);
    return;
  }
  const uint32_t* b = (const uint32_t*)wt + rec * (32 * bits);
  const uint32_t off = 8u - (1u << (bits - 1));
  out[0] = out[1] = out[2] = out[3] = 0u;
  for (int v = 0; v < 32; ++v) {
    uint32_t n = (b[2 * lane + v / 16] >> (2 * (v % 16))) & 3u;
    if (bits == 3) n |= ((b[64 + lane] >> v) & 1u) << 2;
    out[v / 8] |= (n + off) << (4 * (v % 8));
  }
}

/* w4_gemv.cu:112-114: nibble -> fp32 (q) exactly */
static float nib(uint32_t w, int i) {
  uint32_t u = 0x4B000000u | ((w >> (4 * i)) & 0xFu);
  float f;
  memcpy(&f, &u, 4);
  return f - 8388616.0f;
}

int ora_dequant_kt_rows(int bits, const uint8_t* wt, const uint16_t* st, uint16_t* w, int n, int k, int group, int r0,
                        int nr) {
  if (!group_ok(k, group) || k % 32 != 0 || r0 < 0 || nr < 1 || r0 + nr > n) return 1;
  const int SPT = 1024 / group, CPG = group / 32, tiles = kpad(k) >> 10, kc = k >> 5;
  for (int t = 0; t < tiles; ++t)
    for (int o = 0; o < nr; ++o) {
      const size_t rec = (size_t)t * n + r0 + o;
      for (int lane = 0; lane < 32; ++lane) {
        const int c = t * 32 + lane;
        if (c >= kc) continue;
        uint32_t q[4];
        ora_kt_chunk(bits, wt, rec, lane, q);
        const float s = ora_bf2f(st[rec * SPT + lane / CPG]);
        for (int j = 0; j < 4; ++j)
          for (int i = 0; i < 8; ++i) w[(size_t)o * k + (size_t)c * 32 + 8 * j + i] = ora_f2bf(nib(q[j], i) * s);
      }
    }
  return 0;
}

/* ------------------------------------------------------------------------------------------------ GEMV refs */
typedef struct {
  const uint16_t* x;
  int m;
  const uint32_t* packed;
  const uint16_t* scales;
  float* y;
  int ldy, n, k, group, r0, r1;
} RefJob;

static void ref_rows(const RefJob* J) {
  const int k = J->k, G = J->group, groups = k / G;
  int8_t* q = (int8_t*)malloc((size_t)k);
  float* xf = (float*)malloc(sizeof(float) * (size_t)k * J->m);
  for (size_t i = 0; i < (size_t)k * J->m; ++i) xf[i] = ora_bf2f(J->x[i]);
  for (int o = J->r0; o < J->r1; ++o) {
    ora_unpack_row(J->packed + (size_t)o * (k / 8), k, q);
    for (int j = 0; j < J->m; ++j) {
      const float* xr = xf + (size_t)j * k;
      float acc = 0.f;
      for (int g = 0; g < groups; ++g) {
        float ga = 0.f;
        for (int i = g * G; i < (g + 1) * G; ++i) ga += xr[i] * (float)q[i];
        acc += ga * ora_bf2f(J->scales[(size_t)o * groups + g]);
      }
      J->y[(size_t)j * J->ldy + o] = acc;
    }
  }
  free(q);
  free(xf);
}
static void* ref_thread(void* p) {
  ref_rows((const RefJob*)p);
  return NULL;
}

void ora_gemv_ref_f32(const uint16_t* x, int m, const uint32_t* packed, const uint16_t* scales, float* y, int ldy,
                      int n, int k, int group, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > n) nthreads = n;
  RefJob* jobs = (RefJob*)malloc(sizeof(RefJob) * nthreads);
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * nthreads);
  for (int i = 0; i < nthreads; ++i) {
    RefJob J = {x, m, packed, scales, y, ldy, n, k, group, (int)((long)n * i / nthreads),
                (int)((long)n * (i + 1) / nthreads)};
    jobs[i] = J;
  }
  if (nthreads == 1) {
    ref_rows(&jobs[0]);
  } else {
    for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, ref_thread, &jobs[i]);
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
  }
  free(jobs);
  free(th);
}

void ora_gemv_ref_f64(const uint16_t* x, int m, const uint32_t* packed, const uint16_t* scales, double* y,
                      double* mag, int ldy, int n, int k, int group) {
  const int groups = k / group;
  int8_t* q = (int8_t*)malloc((size_t)k);
  for (int o = 0; o < n; ++o) {
    ora_unpack_row(packed + (size_t)o * (k / 8), k, q);
    for (int j = 0; j < m; ++j) {
      double acc = 0.0, a = 0.0;
      for (int i = 0; i < k; ++i) {
        const double t = (double)ora_bf2f(x[(size_t)j * k + i]) * (double)q[i] *
                         (double)ora_bf2f(scales[(size_t)o * groups + i / group]);
        acc += t;
        a += fabs(t);
      }
      y[(size_t)j * ldy + o] = acc;
      mag[(size_t)j * ldy + o] = a;
    }
  }
  free(q);
}

/* w4_gemv.cu:117-127 dot8 and :198-209 dot8w (bf16-rounded weights) */
static float dot8(uint32_t w, const float* xv, int bw, float sc) {
  float s = 0.f;
  for (int i = 0; i < 8; ++i) {
    float q = nib(w, i);
    if (bw) q = ora_bf2f(ora_f2bf(q * sc));
    s = fmaf(xv[i], q, s);
  }
  return s;
}

void ora_gemv_exact_kt(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y,
                       int ldy, int n, int k, int group, int bf16w) {
  ora_gemv_exact_kt_rows(bits, x, m, wt, st, y, ldy, n, k, group, bf16w, 0, n);
}

void ora_gemv_exact_kt_rows(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y,
                            int ldy, int n, int k, int group, int bf16w, int r0, int r1) {
  const int SPT = 1024 / group, CPG = group / 32, tiles = kpad(k) >> 10, kc = k >> 5;
  for (int o = r0; o < r1; ++o)
    for (int j = 0; j < m; ++j) {
      float acc[32];
      for (int l = 0; l < 32; ++l) acc[l] = 0.f;
      for (int t = 0; t < tiles; ++t) {
        const size_t rec = (size_t)t * n + o;
        for (int l = 0; l < 32; ++l) {
          const int c = t * 32 + l;
          float xv[32];
          for (int i = 0; i < 32; ++i) xv[i] = c < kc ? ora_bf2f(x[(size_t)j * k + (size_t)c * 32 + i]) : 0.f;
          uint32_t w[4];
          ora_kt_chunk(bits, wt, rec, l, w);
          const float s = ora_bf2f(st[rec * SPT + l / CPG]);
          const float d = dot8(w[0], xv, bf16w, s) + dot8(w[1], xv + 8, bf16w, s) + dot8(w[2], xv + 16, bf16w, s) +
                          dot8(w[3], xv + 24, bf16w, s);
          acc[l] = bf16w ? acc[l] + d : fmaf(d, s, acc[l]);
        }
      }
      for (int off = 16; off > 0; off >>= 1) {
        float nx[32];
        for (int l = 0; l < 32; ++l) nx[l] = acc[l] + acc[l ^ off];
        memcpy(acc, nx, sizeof(acc));
      }
      y[(size_t)j * ldy + o] = ora_f2bf(acc[0]);
    }
}

/* ------------------------------------------------------------------------------------------------ fast numerics */
static int bf16_expf(uint16_t b) { return (b >> 7) & 0xFF; }

/* q values of KT row o, inputs [0, kp) (padding q = 0) */
static void kt_row_q(int bits, const uint8_t* wt, int n, int k, int o, int8_t* q) {
  const int tiles = kpad(k) >> 10;
  for (int t = 0; t < tiles; ++t)
    for (int l = 0; l < 32; ++l) {
      uint32_t w[4];
      ora_kt_chunk(bits, wt, (size_t)t * n + o, l, w);
      for (int i = 0; i < 32; ++i) q[(size_t)t * 1024 + 32 * l + i] = (int8_t)((int)((w[i >> 3] >> (4 * (i & 7))) & 0xFu) - 8);
    }
}

/* Activation limbs of one group: E = largest bf16 exponent field, x_int = trunc(x * 2^(148 - E)) (exact in double),
 * split into balanced signed bytes x_int = d2 * 2^16 + d1 * 2^8 + d0; returns the three limb sums of d_j * q. */
static void group_limb_sums(const uint16_t* xr, const int8_t* q, int k, int g0, int group, int* E, long long D[3]) {
  int e = 0;
  for (int i = g0; i < g0 + group; ++i)
    if (i < k && bf16_expf(xr[i]) > e) e = bf16_expf(xr[i]);
  D[0] = D[1] = D[2] = 0;
  for (int i = g0; i < g0 + group; ++i) {
    if (i >= k) continue;
    long long xi;
    if (e == 255) /* a non-finite group: an Inf counts as its sign, every other input (finite or NaN) as 0 */
      xi = (xr[i] & 0x7FFF) == 0x7F80 ? ((xr[i] & 0x8000) ? -1 : 1) : 0;
    else
      xi = (long long)ldexp((double)ora_bf2f(xr[i]), 148 - e); /* truncation toward zero */
    const long long x1 = (xi + 128) >> 8, x2 = (x1 + 128) >> 8;           /* arithmetic shifts */
    const long long d0 = xi - x1 * 256, d1 = x1 - x2 * 256, d2 = x2;
    D[0] += d0 * q[i];
    D[1] += d1 * q[i];
    D[2] += d2 * q[i];
  }
  *E = e;
}

/* The activation scale of a group with largest exponent field E: 2^(E - 148); a group holding a NaN: NaN; one holding
 * an Inf and no NaN: +Inf (with its Inf inputs counted as +-1 above, the group adds S * scale * Inf, S the sum of
 * sign(x) * q over them: +-Inf, or NaN where S = 0). */
static float act_scale(const uint16_t* xr, int k, int g0, int group, int E) {
  if (E < 255) return ldexpf(1.0f, E - 148);
  for (int i = g0; i < g0 + group && i < k; ++i)
    if ((xr[i] & 0x7FFF) > 0x7F80) return NAN;
  return INFINITY;
}

static long long group_sum(const uint16_t* xr, const int8_t* q, int k, int g0, int group, int* E) {
  long long D[3];
  group_limb_sums(xr, q, k, g0, group, E, D);
  return D[2] * 65536 + D[1] * 256 + D[0];
}

long long ora_fast_group_sum(int bits, const uint16_t* x, const uint8_t* wt, int n, int k, int group, int o, int g,
                             int* E) {
  int8_t* q = (int8_t*)malloc((size_t)kpad(k));
  kt_row_q(bits, wt, n, k, o, q);
  const long long r = group_sum(x, q, k, g * group, group, E);
  free(q);
  return r;
}

void ora_gemv_fast_kt(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y, int ldy,
                      int n, int k, int group) {
  ora_gemv_fast_kt_rows(bits, x, m, wt, st, y, ldy, n, k, group, 0, n);
}

void ora_gemv_fast_kt_rows(int bits, const uint16_t* x, int m, const uint8_t* wt, const uint16_t* st, uint16_t* y,
                           int ldy, int n, int k, int group, int r0, int r1) {
  const int kp = kpad(k), SPT = 1024 / group, ngroups = kp / group, nquad = ngroups / 4;
  const int nt = kp / 1024, qpt = nquad / nt, P = nt < 8 ? nt : 8;
  int8_t* q = (int8_t*)malloc((size_t)kp);
  for (int o = r0; o < r1; ++o) {
    kt_row_q(bits, wt, n, k, o, q);
    for (int j = 0; j < m; ++j) {
      const uint16_t* xr = x + (size_t)j * k;
      float acc[8][4];
      memset(acc, 0, sizeof(acc));
      for (int qd = 0, p = 0; qd < nquad; ++qd) {
        while (qd >= qpt * ((p + 1) * nt / P)) ++p; /* stripe p = tiles [p * nt / P, (p + 1) * nt / P) */
        for (int s = 0; s < 4; ++s) {
          const int g = 4 * qd + s, t = g * group / 1024, gi = g % SPT;
          int E;
          long long D[3];
          group_limb_sums(xr, q, k, g * group, group, &E, D);
          const int T = (int)(D[2] * 256 + D[1]);
          const float gsum = fmaf((float)T, 256.0f, (float)D[0]);
          const float sE = ora_bf2f(st[((size_t)t * n + o) * SPT + gi]) * act_scale(xr, k, g * group, group, E);
          acc[p][s] = fmaf(gsum, sE, acc[p][s]);
        }
      }
      float yv = 0.f;
      for (int p = 0; p < P; ++p) {
        const float part = ((acc[p][0] + acc[p][1]) + acc[p][2]) + acc[p][3];
        yv = p == 0 ? part : yv + part;
      }
      y[(size_t)j * ldy + o] = ora_f2bf(yv);
    }
  }
  free(q);
}

/* ------------------------------------------------------------------------------------------------ generators */
uint32_t ora_xorshift32(uint32_t* s) {
  uint32_t v = *s;
  v ^= v << 13, v ^= v >> 17, v ^= v << 5;
  *s = v;
  return v;
}

/* splitmix64 finaliser of (seed, index) */
uint32_t ora_hash_u32(uint64_t seed, uint64_t index) {
  uint64_t z = seed * 0x9E3779B97F4A7C15ull + index * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return (uint32_t)((z ^ (z >> 31)) >> 16);
}

static double normal_at(uint64_t seed, uint64_t i) {
  const double u1 = ((double)ora_hash_u32(seed, 2 * i) + 1.0) / 4294967296.0;
  const double u2 = (double)ora_hash_u32(seed, 2 * i + 1) / 4294967296.0;
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void ora_gen_container(uint64_t seed, int n, int k, int lo, int span, uint32_t* packed) {
  const size_t words = (size_t)n * k / 8;
  for (size_t w = 0; w < words; ++w) {
    uint32_t v = 0;
    for (int j = 0; j < 8; ++j) {
      const int q = lo + (int)(ora_hash_u32(seed, 8 * w + j) % (uint32_t)span);
      v |= (uint32_t)(q + 8) << (4 * j);
    }
    packed[w] = v;
  }
}

void ora_gen_scales(uint64_t seed, size_t count, float sa, float sb, uint16_t* s) {
  for (size_t i = 0; i < count; ++i) s[i] = ora_f2bf((float)(fabs(normal_at(seed, i)) * sa + sb));
}

void ora_gen_x(uint64_t seed, size_t count, float xs, uint16_t* x) {
  for (size_t i = 0; i < count; ++i) x[i] = ora_f2bf((float)(normal_at(seed, i) * xs));
}

/* ------------------------------------------------------------------------------------------------ adjacent GEMVs */
/* kernels/src/i8_gemv.cu:28-70: the warp of row o (32 lanes), lane l over chunks l, l + 32, ...; per chunk a 16-input
 * fmaf chain from 0 (dot4 x 4, inputs in order), added to the lane's sum; then the xor butterfly and the row scale */
void ora_i8_gemv(const uint16_t* x, const int8_t* q, const float* scale, uint16_t* y, int m, int n, int k, int ldy) {
  const int chunks = k / 16;
  for (int o = 0; o < n; ++o) {
    const int8_t* w = q + (size_t)o * k;
    for (int j = 0; j < m; ++j) {
      const uint16_t* xr = x + (size_t)j * k;
      float v[32];
      for (int l = 0; l < 32; ++l) {
        float acc = 0.f;
        for (int c = l; c < chunks; c += 32) {
          float s = 0.f;
          for (int e = 0; e < 16; ++e) s = fmaf(ora_bf2f(xr[16 * c + e]), (float)w[16 * c + e], s);
          acc += s;
        }
        v[l] = acc;
      }
      for (int d = 16; d > 0; d >>= 1) {
        float t[32];
        for (int l = 0; l < 32; ++l) t[l] = v[l] + v[l ^ d];
        memcpy(v, t, sizeof(v));
      }
      y[(size_t)j * ldy + o] = ora_f2bf(v[0] * scale[o]);
    }
  }
}
