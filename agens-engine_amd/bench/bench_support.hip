// Benchmark support for bench.py (not part of the product ABI): device-side synthetic data in the reference's int4
// container, a stream-read ceiling probe, and a native launcher that replays a list of GEMV launches (eager or as
// one captured hipGraph) and times it with HIP events on its own stream.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "agens_kernels.h"

namespace {

__device__ __forceinline__ uint32_t mix(uint64_t seed, uint64_t index) {
  uint64_t z = seed * 0x9E3779B97F4A7C15ull + index * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return (uint32_t)((z ^ (z >> 31)) >> 16);
}

__device__ __forceinline__ float normal(uint64_t seed, uint64_t i) {
  const float u1 = ((float)mix(seed, 2 * i) + 1.0f) * 2.3283064e-10f;
  const float u2 = (float)mix(seed, 2 * i + 1) * 2.3283064e-10f;
  return sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
}

__device__ __forceinline__ uint16_t to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__global__ void gen_container_kernel(uint64_t seed, size_t words, int lo, int span, uint32_t* p) {
  for (size_t w = blockIdx.x * (size_t)blockDim.x + threadIdx.x; w < words; w += (size_t)gridDim.x * blockDim.x) {
    const uint32_t h0 = mix(seed, 2 * w), h1 = mix(seed, 2 * w + 1);
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t r = ((j < 4 ? h0 : h1) >> (8 * (j & 3))) & 0xFFu;  // 8 random bits per code
      const int q = lo + (int)((r * (uint32_t)span) >> 8);
      v |= (uint32_t)(q + 8) << (4 * j);
    }
    p[w] = v;
  }
}

__global__ void gen_scales_kernel(uint64_t seed, size_t count, float sa, float sb, uint16_t* s) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x)
    s[i] = to_bf16(fabsf(normal(seed, i)) * sa + sb);
}

__global__ void gen_x_kernel(uint64_t seed, size_t count, float xs, uint16_t* x) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x)
    x[i] = to_bf16(normal(seed, i) * xs);
}

__global__ void gen_i8_kernel(uint64_t seed, size_t words, uint32_t* q) {  // uniform int8 bytes
  for (size_t w = blockIdx.x * (size_t)blockDim.x + threadIdx.x; w < words; w += (size_t)gridDim.x * blockDim.x)
    q[w] = mix(seed, w) ^ (mix(seed + 1, w) << 16);
}

__global__ void gen_f32_kernel(uint64_t seed, size_t count, float sa, float sb, float* s) {  // |N(0,1)| sa + sb
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x)
    s[i] = fabsf(normal(seed, i)) * sa + sb;
}

__global__ void read_kernel(const uint4* __restrict__ p, size_t n16, uint32_t* out) {
  uint32_t acc = 0;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p + i));
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) out[0] = acc;
}

__global__ void copy_kernel(const uint4* __restrict__ a, uint4* __restrict__ b, size_t n16) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    b[i] = a[i];
}

unsigned grid_for(size_t items) {
  const size_t b = (items + 255) / 256;
  return (unsigned)(b < 8192 ? (b ? b : 1) : 8192);
}

}  // namespace

extern "C" {

struct AgbLaunch {
  int bits, m, nseg, k, group, bf16w;
  const void* x;
  const void* wt[4];
  const void* st[4];
  void* y[4];
  int n[4];
  int ldy[4];
  int use_ldy;
  int pad;
};

int agb_gen_container(uint64_t seed, int n, int k, int lo, int span, void* packed, void* stream) {
  const size_t words = (size_t)n * k / 8;
  hipLaunchKernelGGL(gen_container_kernel, dim3(grid_for(words)), dim3(256), 0, (hipStream_t)stream, seed, words, lo,
                     span, (uint32_t*)packed);
  return (int)hipGetLastError();
}

int agb_gen_scales(uint64_t seed, size_t count, float sa, float sb, void* s, void* stream) {
  hipLaunchKernelGGL(gen_scales_kernel, dim3(grid_for(count)), dim3(256), 0, (hipStream_t)stream, seed, count, sa, sb,
                     (uint16_t*)s);
  return (int)hipGetLastError();
}

int agb_gen_x(uint64_t seed, size_t count, float xs, void* x, void* stream) {
  hipLaunchKernelGGL(gen_x_kernel, dim3(grid_for(count)), dim3(256), 0, (hipStream_t)stream, seed, count, xs,
                     (uint16_t*)x);
  return (int)hipGetLastError();
}

int agb_gen_i8(uint64_t seed, size_t bytes, void* q, void* stream) {  // bytes % 4 == 0
  hipLaunchKernelGGL(gen_i8_kernel, dim3(grid_for(bytes / 4)), dim3(256), 0, (hipStream_t)stream, seed, bytes / 4,
                     (uint32_t*)q);
  return (int)hipGetLastError();
}

int agb_gen_f32(uint64_t seed, size_t count, float sa, float sb, void* s, void* stream) {
  hipLaunchKernelGGL(gen_f32_kernel, dim3(grid_for(count)), dim3(256), 0, (hipStream_t)stream, seed, count, sa, sb,
                     (float*)s);
  return (int)hipGetLastError();
}

// ak_bf16_gemv_bi over `ncopies` weight copies in turn (w + c * n * k), timed as agb_time_i8_gemv
int agb_time_bi_gemv(const void* x, const void* w, void* y, int m, int n, int k, int ncopies, int warmup, int steps,
                     float* ms) {
  hipStream_t s;
  int e = (int)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e) return e;
  auto one = [&](int i) {
    return ak_bf16_gemv_bi(x, (const uint16_t*)w + (size_t)(i % ncopies) * n * k, nullptr, y, m, n, k, s);
  };
  for (int i = 0; i < warmup && !e; ++i) e = one(i);
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  bool cap = false;
  if (!e) {
    e = (int)hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    cap = !e;
  }
  for (int i = 0; i < steps && !e; ++i) e = one(i);
  if (cap) {
    const int e2 = (int)hipStreamEndCapture(s, &g);
    if (!e) e = e2;
  }
  if (!e) e = (int)hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  if (!e) e = (int)hipGraphLaunch(ge, s);
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  if (!e) e = (int)hipEventRecord(a, s);
  if (!e) e = (int)hipGraphLaunch(ge, s);
  if (!e) e = (int)hipEventRecord(b, s);
  if (!e) e = (int)hipEventSynchronize(b);
  float t = 0.f;
  if (!e) e = (int)hipEventElapsedTime(&t, a, b);
  *ms = t / steps;
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (ge) hipGraphExecDestroy(ge);
  if (g) hipGraphDestroy(g);
  hipStreamSynchronize(s);
  hipStreamDestroy(s);
  return e;
}

// ak_i8_gemv over `ncopies` weight copies in turn (w + c * n * k, scale + c * n), `steps` launches captured in one
// hipGraph after `warmup` eager ones; *ms = the mean time per launch (HIP events on the launching stream).
int agb_time_i8_gemv(const void* x, const void* w, const void* scale, void* y, int m, int n, int k, int ncopies,
                     int warmup, int steps, float* ms) {
  hipStream_t s;
  int e = (int)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e) return e;
  auto one = [&](int i) {
    const int c = i % ncopies;
    return ak_i8_gemv(x, (const int8_t*)w + (size_t)c * n * k, (const float*)scale + (size_t)c * n, y, m, n, k, n, s);
  };
  for (int i = 0; i < warmup && !e; ++i) e = one(i);
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  bool cap = false;
  if (!e) {
    e = (int)hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    cap = !e;
  }
  for (int i = 0; i < steps && !e; ++i) e = one(i);
  if (cap) {
    const int e2 = (int)hipStreamEndCapture(s, &g);
    if (!e) e = e2;
  }
  if (!e) e = (int)hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  if (!e) e = (int)hipGraphLaunch(ge, s);  // first replay untimed
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  if (!e) e = (int)hipEventRecord(a, s);
  if (!e) e = (int)hipGraphLaunch(ge, s);
  if (!e) e = (int)hipEventRecord(b, s);
  if (!e) e = (int)hipEventSynchronize(b);
  float t = 0.f;
  if (!e) e = (int)hipEventElapsedTime(&t, a, b);
  *ms = t / steps;
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (ge) hipGraphExecDestroy(ge);
  if (g) hipGraphDestroy(g);
  hipStreamSynchronize(s);
  hipStreamDestroy(s);
  return e;
}

static int launch_one(const AgbLaunch& L, hipStream_t s) {
  return ak_wq_gemv_kt_multi(L.bits, L.x, L.m, L.nseg, L.wt, L.st, L.y, L.n, L.use_ldy ? L.ldy : nullptr, L.k,
                             L.group, L.bf16w, s);
}

// Replays plan[0..nlaunch) `warmup` times untimed, then `steps` times between two events; *ms = elapsed / steps.
// use_graph: the plan is captured once into a hipGraph (after the warmup) and each step is one graph launch.
int agb_run(const AgbLaunch* plan, int nlaunch, int warmup, int steps, int use_graph, float* ms) {
  hipStream_t s;
  int e = (int)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e) return e;
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  hipGraphExec_t ge = nullptr;
  hipGraph_t g = nullptr;
  for (int w = 0; w < (warmup > 0 ? warmup : 1) && !e; ++w)
    for (int i = 0; i < nlaunch && !e; ++i) e = launch_one(plan[i], s);
  if (!e) e = (int)hipStreamSynchronize(s);
  if (!e && use_graph) {
    e = (int)hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    for (int i = 0; i < nlaunch && !e; ++i) e = launch_one(plan[i], s);
    const int e2 = (int)hipStreamEndCapture(s, &g);
    if (!e) e = e2;
    if (!e) e = (int)hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (!e) e = (int)hipGraphLaunch(ge, s);
    if (!e) e = (int)hipStreamSynchronize(s);
  }
  if (!e) {
    hipEventRecord(a, s);
    for (int st = 0; st < steps && !e; ++st) {
      if (use_graph) e = (int)hipGraphLaunch(ge, s);
      else
        for (int i = 0; i < nlaunch && !e; ++i) e = launch_one(plan[i], s);
    }
    hipEventRecord(b, s);
    if (!e) e = (int)hipEventSynchronize(b);
    float t = 0.f;
    if (!e) e = (int)hipEventElapsedTime(&t, a, b);
    *ms = steps > 0 ? t / steps : 0.f;
  }
  if (ge) hipGraphExecDestroy(ge);
  if (g) hipGraphDestroy(g);
  hipEventDestroy(a);
  hipEventDestroy(b);
  hipStreamSynchronize(s);
  hipStreamDestroy(s);
  return e;
}

// The plan as one chain (ak_wq_chain_*: every step waits for the one before it, as in a decode step where each linear
// reads the previous one's output): `warmup` untimed runs, then `steps` runs between two events (one graph launch
// each with use_graph).  *chained = 1 if the chain ran as one chained launch; *status = ak_wq_chain_status().
int agb_run_chain_ex(const AgbLaunch* plan, int nlaunch, int warmup, int steps, int use_graph, float* ms, int* chained,
                     int* status, int independent);
int agb_run_chain(const AgbLaunch* plan, int nlaunch, int warmup, int steps, int use_graph, float* ms, int* chained,
                  int* status) {
  return agb_run_chain_ex(plan, nlaunch, warmup, steps, use_graph, ms, chained, status, 0);
}
// independent = 1: every step declared independent of the others (no grid barriers; the caller gives every step its
// own outputs): the streaming bound of the chained kernel without the decode data flow
int agb_run_chain_ex(const AgbLaunch* plan, int nlaunch, int warmup, int steps, int use_graph, float* ms, int* chained,
                     int* status, int independent) {
  std::vector<ak_wq_step> st((size_t)nlaunch);
  for (int i = 0; i < nlaunch; ++i) {
    const AgbLaunch& L = plan[i];
    ak_wq_step& d = st[(size_t)i];
    memset(&d, 0, sizeof(d));
    d.bits = L.bits, d.m = L.m, d.nseg = L.nseg, d.k = L.k, d.group = L.group, d.bf16w = L.bf16w, d.x = L.x;
    for (int j = 0; j < L.nseg; ++j) {
      d.wt[j] = L.wt[j], d.st[j] = L.st[j], d.y[j] = L.y[j], d.n[j] = L.n[j];
      d.ldy[j] = L.use_ldy ? L.ldy[j] : 0;
    }
    d.independent = independent;
  }
  void* ch = nullptr;
  int e = ak_wq_chain_create(st.data(), nlaunch, &ch);
  if (e) return e;
  *chained = ak_wq_chain_chained(ch);
  hipStream_t s;
  e = (int)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e) {
    ak_wq_chain_destroy(ch);
    return e;
  }
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  hipGraphExec_t ge = nullptr;
  hipGraph_t g = nullptr;
  for (int w = 0; w < (warmup > 0 ? warmup : 1) && !e; ++w) e = ak_wq_chain_run(ch, s);
  if (!e) e = (int)hipStreamSynchronize(s);
  if (!e && use_graph) {
    e = (int)hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (!e) e = ak_wq_chain_run(ch, s);
    const int e2 = (int)hipStreamEndCapture(s, &g);
    if (!e) e = e2;
    if (!e) e = (int)hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (!e) e = (int)hipGraphLaunch(ge, s);
    if (!e) e = (int)hipStreamSynchronize(s);
  }
  if (!e) {
    hipEventRecord(a, s);
    for (int r = 0; r < steps && !e; ++r) e = use_graph ? (int)hipGraphLaunch(ge, s) : ak_wq_chain_run(ch, s);
    hipEventRecord(b, s);
    if (!e) e = (int)hipEventSynchronize(b);
    float t = 0.f;
    if (!e) e = (int)hipEventElapsedTime(&t, a, b);
    *ms = steps > 0 ? t / steps : 0.f;
  }
  *status = ak_wq_chain_status();
  if (ge) hipGraphExecDestroy(ge);
  if (g) hipGraphDestroy(g);
  hipEventDestroy(a);
  hipEventDestroy(b);
  hipStreamSynchronize(s);
  hipStreamDestroy(s);
  ak_wq_chain_destroy(ch);
  return e;
}

// Duration of every launch of the plan (average over `reps` passes), each bracketed by its own pair of events on the
// launching stream; ms_each[i] in milliseconds.
int agb_time_each(const AgbLaunch* plan, int nlaunch, int reps, float* ms_each) {
  hipStream_t s;
  int e = (int)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e) return e;
  std::vector<hipEvent_t> ev(2 * (size_t)nlaunch);
  for (auto& x : ev) hipEventCreate(&x);
  for (int i = 0; i < nlaunch; ++i) ms_each[i] = 0.f;
  for (int r = 0; r < reps && !e; ++r) {
    for (int i = 0; i < nlaunch && !e; ++i) {
      hipEventRecord(ev[2 * i], s);
      e = launch_one(plan[i], s);
      hipEventRecord(ev[2 * i + 1], s);
    }
    if (!e) e = (int)hipStreamSynchronize(s);
    for (int i = 0; i < nlaunch && !e; ++i) {
      float t = 0.f;
      e = (int)hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]);
      ms_each[i] += t / reps;
    }
  }
  for (auto& x : ev) hipEventDestroy(x);
  hipStreamDestroy(s);
  return e;
}

// Stream-read ceiling: 16-byte nontemporal loads over `bytes` (>= 1 GB beats the 256 MB last-level cache).
int agb_read_bw(size_t bytes, int reps, float* gbps) {
  void* buf = nullptr;
  void* sink = nullptr;
  int e = (int)hipMalloc(&buf, bytes);
  if (!e) e = (int)hipMalloc(&sink, 16);
  if (!e) e = (int)hipMemset(buf, 1, bytes);
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  float best = 0.f;
  for (int blocks : {2048, 4096}) {
    if (e) break;
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(512), 0, 0, (const uint4*)buf, bytes / 16, (uint32_t*)sink);
    hipEventRecord(a, 0);
    for (int r = 0; r < reps; ++r)
      hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(512), 0, 0, (const uint4*)buf, bytes / 16, (uint32_t*)sink);
    hipEventRecord(b, 0);
    e = (int)hipEventSynchronize(b);
    float t = 0.f;
    hipEventElapsedTime(&t, a, b);
    const float g = (float)((double)bytes * reps / (t * 1e6));
    if (g > best) best = g;
  }
  *gbps = best;
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (buf) hipFree(buf);
  if (sink) hipFree(sink);
  return e;
}

// A plain copy of `bytes` (read + write), the calibration kernel for the HBM traffic counters.
int agb_copy(size_t bytes, int reps) {
  void *a = nullptr, *b = nullptr;
  int e = (int)hipMalloc(&a, bytes);
  if (!e) e = (int)hipMalloc(&b, bytes);
  if (!e) e = (int)hipMemset(a, 3, bytes);
  for (int r = 0; r < reps && !e; ++r) {
    hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, 0, (const uint4*)a, (uint4*)b, bytes / 16);
    e = (int)hipGetLastError();
  }
  if (!e) e = (int)hipDeviceSynchronize();
  if (a) hipFree(a);
  if (b) hipFree(b);
  return e;
}

// The GEMV-versus-GEMM crossover: `steps` eager calls on one stream after `warmup`, weights rotated over `ncopies`
// KT copies (wts[c], sts[c]); *ms = the mean time per call (HIP events).
//   mode 0: ak_wq_gemv_kt_multi (the quantized GEMV, m <= 128);
//   mode 1: ak_wq_dequant_kt_rows of all n rows into wdense, then ak_bf16_linear_f32reduce (the prefill route).
int agb_time_xover(int bits, const void* x, int m, const void* const* wts, const void* const* sts, int ncopies,
                   void* wdense, void* y, int n, int k, int mode, int warmup, int steps, float* ms) {
  hipStream_t s;
  int e = (int)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e) return e;
  auto one = [&](int i) {
    const void* w = wts[i % ncopies];
    const void* sc = sts[i % ncopies];
    if (mode == 0) {
      void* yy = y;
      return ak_wq_gemv_kt_multi(bits, x, m, 1, &w, &sc, &yy, &n, nullptr, k, 128, 0, s);
    }
    if (mode == 2) return ak_wq_gemm_kt(bits, x, m, w, sc, y, n, 0, k, 128, s);  // the fused prefill GEMM
    int r = ak_wq_dequant_kt_rows(bits, w, sc, wdense, n, k, 128, 0, n, s);
    if (!r) r = ak_bf16_linear_f32reduce(x, wdense, y, m, n, k, s);
    return r;
  };
  for (int i = 0; i < warmup && !e; ++i) e = one(i);
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  if (!e) e = (int)hipEventRecord(a, s);
  for (int i = 0; i < steps && !e; ++i) e = one(i);
  if (!e) e = (int)hipEventRecord(b, s);
  if (!e) e = (int)hipEventSynchronize(b);
  float t = 0.f;
  if (!e) e = (int)hipEventElapsedTime(&t, a, b);
  *ms = t / steps;
  hipEventDestroy(a);
  hipEventDestroy(b);
  hipStreamSynchronize(s);
  hipStreamDestroy(s);
  return e;
}

}  // extern "C"
