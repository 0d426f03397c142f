// Host side of the quantized-linear path (see agens_linear.h).
#include "agens_linear.h"

#include <algorithm>
#include <cstring>
#include <mutex>

#include "agens_kernels.h"

namespace agens {

void check(int code, const char* what) {
  if (code == 0) return;
  const char* msg = ak_error_string(code);
  throw Error(std::string(what) + ": error " + std::to_string(code) + " (" + (msg ? msg : "?") + ")");
}

DeviceBuffer::DeviceBuffer(size_t bytes) : bytes_(bytes) {
  check(ak_malloc(&ptr_, bytes ? bytes : 1), "malloc");
}
DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) { o.ptr_ = nullptr; }
DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
  if (this != &o) {
    if (ptr_) ak_free(ptr_);
    ptr_ = o.ptr_, bytes_ = o.bytes_, o.ptr_ = nullptr;
  }
  return *this;
}
DeviceBuffer::~DeviceBuffer() {
  if (ptr_) ak_free(ptr_);
}
void* DeviceBuffer::leak() {
  void* p = ptr_;
  ptr_ = nullptr;
  return p;
}

DeviceBuffer device_alloc(size_t bytes) { return DeviceBuffer(bytes); }

DeviceBuffer upload(const void* host, size_t bytes) {
  DeviceBuffer b(bytes);
  check(ak_memcpy_h2d(b.ptr(), host, bytes), "memcpy_h2d");
  return b;
}

namespace {

void check_sizes(const char* what, const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n,
                 int k, int group) {
  if (n < 1 || k < 1 || group < 1 || packed.size() != (size_t)n * k / 2 ||
      scales.size() != (size_t)n * (k / group) * 2)
    throw Error(std::string(what) + ": " + std::to_string(packed.size()) + " / " + std::to_string(scales.size()) +
                " bytes for [" + std::to_string(n) + ", " + std::to_string(k) + "] group " + std::to_string(group));
}

// repack through the C ABI; returns its code (1: a value outside `bits` bits, or bad arguments)
int repack(int bits, const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n, int k, int group,
           KtPair& out) {
  DeviceBuffer p = upload(packed.data(), packed.size()), s = upload(scales.data(), scales.size());
  out.first = device_alloc(ak_wq_kt_weight_bytes(bits, n, k));
  out.second = device_alloc(ak_w4_kt_scale_bytes(n, k, group));
  const int e = ak_wq_repack_kt(bits, static_cast<const int32_t*>(p.ptr()), s.ptr(), out.first.ptr(),
                                out.second.ptr(), n, k, group, nullptr);
  // the staging buffers are freed when p and s go out of scope: wait for the repack to have read them
  const int e2 = ak_synchronize();
  return e ? e : e2;
}

}  // namespace

KtPair w4_upload_kt(const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n, int k, int group) {
  check_sizes("w4_upload_kt", packed, scales, n, k, group);
  KtPair out;
  check(repack(4, packed, scales, n, k, group, out), "w4_repack_kt");
  return out;
}

std::optional<KtPair> w3_upload_kt(const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n,
                                   int k, int group) {
  check_sizes("w3_upload_kt", packed, scales, n, k, group);
  KtPair out;
  const int e = repack(3, packed, scales, n, k, group, out);
  if (e == 1) return std::nullopt;  // a 4-bit value
  check(e, "w3_repack_kt");
  return out;
}

KtPair wq_upload_kt(int bits, const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n, int k,
                    int group) {
  if (bits == 4) return w4_upload_kt(packed, scales, n, k, group);
  check_sizes("wq_upload_kt", packed, scales, n, k, group);
  KtPair out;
  const int e = repack(bits, packed, scales, n, k, group, out);
  if (e == 1)
    throw Error("wq_upload_kt: [" + std::to_string(n) + ", " + std::to_string(k) + "] has values outside " +
                std::to_string(bits) + " bits");
  check(e, "wq_repack_kt");
  return out;
}

namespace {
size_t g_tile_bytes = (size_t)64 << 20;  // bound of the dequantized tile (the reference's S.wdq / g_w4_tile_bytes)
std::mutex g_wdq_mu;
void* g_wdq = nullptr;  // the process's dequantization scratch (grown on demand, held for the process)
size_t g_wdq_bytes = 0;

// output rows per prefill tile (m1_model.cu:1822-1826): multiples of 256 within the tile bound, at least 256
int tile_rows(int k, int n) {
  const long r = (long)(g_tile_bytes / ((size_t)k * 2)) & ~255L;
  return (int)std::max(256L, std::min<long>(r, n));
}
}  // namespace

void set_prefill_tile_bytes(size_t bytes) { g_tile_bytes = bytes; }

namespace {
int g_prefill_route = -1;  // -1: by shape, 0: dequantized tiles x library GEMM, 1: the fused GEMM

// The fused prefill GEMM (ak_wq_gemm_kt) against dequantized tiles x rocBLAS, measured on MI355X (us per call,
// bench.py --config prefill and --config xover):
//   gate_up W3 55296 x 5120:   m = 512: 441 vs 448, m = 2048: 1436 vs 987;
//   LM head W4 152064 x 5120:  m = 512: 934 vs 1092, m = 2048: 3076 vs 2648;
//   down W2 5120 x 27648:      m = 512: 239 vs 354, m = 2048: 677 vs 516;
//   o W4 5120 x 5120:          m = 256:  41 vs  59, m = 512:  58 vs  51;
//   qkv W4 7168 x 5120:        m = 256:  49 vs  85, m = 512:  70 vs  72.
// The fused kernel wins on long k and on wide linears up to several hundred tokens and on every linear up to 256
// tokens (narrow ones split k across workgroups); the library GEMM on narrow short-k linears beyond that and at large
// m (the fused kernel expands every weight once per token tile).
bool prefill_fused(int n, int k, int m) {
  if (g_prefill_route >= 0) return g_prefill_route == 1;
  return m <= 256 || (k >= 16384 && m <= 1024) || (n >= 16384 && m <= (n >= 100000 ? 1024 : 512));
}
}  // namespace

void set_prefill_route(int mode) { g_prefill_route = mode < 0 ? -1 : (mode ? 1 : 0); }

int linear(const QuantLinear& t, const void* x, void* y, int m, int n, int k, int bf16w, void* stream) {
  if (t.n != n || t.k != k || m < 1 || t.np < 1 || t.np > 2) return 1;
  if (m > 128 && prefill_fused(n, k, m)) {
    // prefill through the fused GEMM: one launch per part, straight from the KT weights into its columns of y
    for (int j = 0; j < t.np; ++j) {
      const QuantPart& q = t.p[j];
      if (const int e = ak_wq_gemm_kt(q.bits, x, m, q.wt, q.st, static_cast<uint16_t*>(y) + q.r0, q.n, n, k, q.group,
                                      stream))
        return e;
    }
    return 0;
  }
  if (m > 128) {
    // prefill (m1_model.cu:1876-1897): dequantize a tile of output rows at a time into the bounded scratch and GEMM
    // that column tile of y (tiles by output row whatever the parts)
    const int tn = tile_rows(k, n);
    std::lock_guard<std::mutex> lock(g_wdq_mu);
    const size_t need = (size_t)std::min(tn, n) * k * 2;
    if (g_wdq_bytes < need) {
      if (g_wdq) ak_free(g_wdq);
      g_wdq = nullptr;
      g_wdq_bytes = 0;
      if (const int e = ak_malloc(&g_wdq, need)) return e;
      g_wdq_bytes = need;
    }
    uint16_t* const wdq = static_cast<uint16_t*>(g_wdq);
    for (int n0 = 0; n0 < n; n0 += tn) {
      const int nt = std::min(tn, n - n0);
      for (int j = 0; j < t.np; ++j) {
        const QuantPart& q = t.p[j];
        const int a0 = std::max(n0, q.r0), a1 = std::min(n0 + nt, q.r0 + q.n);
        if (a0 < a1)
          if (const int e = ak_wq_dequant_kt_rows(q.bits, q.wt, q.st, wdq + (size_t)(a0 - n0) * k, q.n, k, q.group,
                                                  a0 - q.r0, a1 - a0, stream))
            return e;
      }
      if (tn >= n) return ak_bf16_linear_f32reduce(x, wdq, y, m, n, k, stream);
      if (const int e = ak_bf16_linear_f32reduce_ld(x, wdq, static_cast<uint16_t*>(y) + n0, m, nt, k, n, stream))
        return e;
    }
    return 0;
  }
  for (int j = 0; j < t.np; ++j) {
    const QuantPart& q = t.p[j];
    void* yp = static_cast<uint16_t*>(y) + q.r0;
    const void* wt = q.wt;
    const void* st = q.st;
    const int e = ak_wq_gemv_kt_multi(q.bits, x, m, 1, &wt, &st, &yp, &q.n, &n, k, q.group, bf16w, stream);
    if (e) return e;
  }
  return 0;
}

int linear_shared(const void* x, int nl, const QuantLinear* const* lins, void* const* ys, const int* ns, int m, int k,
                  int bf16w, void* stream) {
  bool ok = nl >= 1 && nl <= 4 && m == 1;
  for (int j = 0; j < nl && ok; ++j) ok = lins[j] && lins[j]->np == 1 && lins[j]->n == ns[j] && lins[j]->k == k;
  if (ok) {  // one launch per (bits, group) class
    bool done[4] = {false, false, false, false};
    for (int j = 0; j < nl; ++j) {
      if (done[j]) continue;
      const QuantPart& pj = lins[j]->p[0];
      const void *wt[4], *st[4];
      void* y[4];
      int nn[4], c = 0;
      for (int i = j; i < nl; ++i) {
        const QuantPart& pi = lins[i]->p[0];
        if (done[i] || pi.bits != pj.bits || pi.group != pj.group) continue;
        wt[c] = pi.wt, st[c] = pi.st, y[c] = ys[i], nn[c] = ns[i], ++c, done[i] = true;
      }
      const int e = ak_wq_gemv_kt_multi(pj.bits, x, m, c, wt, st, y, nn, nullptr, k, pj.group, bf16w, stream);
      if (e) return e;
    }
    return 0;
  }
  for (int j = 0; j < nl; ++j) {
    if (!lins[j]) return 1;
    const int e = linear(*lins[j], x, ys[j], m, ns[j], k, bf16w, stream);
    if (e) return e;
  }
  return 0;
}

LinearChain::~LinearChain() {
  if (chain_) ak_wq_chain_destroy(chain_);
}

int LinearChain::push(int bits, int group, const void* x, int m, int k, int nseg, const void* const* wt,
                      const void* const* st, void* const* y, const int* n, const int* ldy, int bf16w,
                      bool independent, bool act) {
  if (chain_ || nseg < 1 || nseg > 4 || m < 1 || m > 128) return 1;
  ak_wq_step s;
  std::memset(&s, 0, sizeof(s));
  s.bits = bits, s.m = m, s.nseg = nseg, s.k = k, s.group = group, s.bf16w = bf16w;
  s.x = x;
  for (int i = 0; i < nseg; ++i) s.wt[i] = wt[i], s.st[i] = st[i], s.y[i] = y[i], s.n[i] = n[i], s.ldy[i] = ldy[i];
  s.independent = independent ? 1 : 0;
  s.act = act ? 1 : 0;
  steps_.push_back(s);
  return 0;
}

int LinearChain::add(const QuantLinear& t, const void* x, void* y, int m, int bf16w, bool independent, bool act) {
  if (chain_ || t.np < 1 || t.np > 2 || m < 1 || m > 128 || (act && t.np != 1)) return 1;
  for (int j = 0; j < t.np; ++j) {
    const QuantPart& q = t.p[j];
    const void* wt = q.wt;
    const void* st = q.st;
    void* yp = static_cast<uint16_t*>(y) + q.r0;
    // the parts of one linear read the same x and write disjoint rows: the second does not wait for the first
    if (const int e = push(q.bits, q.group, x, m, t.k, 1, &wt, &st, &yp, &q.n, &t.n, bf16w, j > 0 || independent, act))
      return e;
  }
  return 0;
}

int LinearChain::add_shared(const void* x, int nl, const QuantLinear* const* lins, void* const* ys, const int* ns,
                            int m, int k, int bf16w, bool independent) {
  if (chain_ || nl < 1 || nl > 4 || !lins || !ys || !ns) return 1;
  for (int j = 0; j < nl; ++j)
    if (!lins[j] || lins[j]->n != ns[j] || lins[j]->k != k) return 1;
  bool done[4] = {false, false, false, false};
  bool first = true;
  for (int j = 0; j < nl; ++j) {
    if (done[j]) continue;
    if (lins[j]->np != 1) {  // a multi-part linear: its own steps
      done[j] = true;
      if (const int e = add(*lins[j], x, ys[j], m, bf16w, !first || independent)) return e;
      first = false;
      continue;
    }
    const QuantPart& pj = lins[j]->p[0];
    const void *wt[4], *st[4];
    void* y[4];
    int nn[4], ld[4], c = 0;
    for (int i = j; i < nl; ++i) {
      if (done[i] || lins[i]->np != 1) continue;
      const QuantPart& pi = lins[i]->p[0];
      if (pi.bits != pj.bits || pi.group != pj.group) continue;
      wt[c] = pi.wt, st[c] = pi.st, y[c] = ys[i], nn[c] = ns[i], ld[c] = ns[i], ++c;
      done[i] = true;
    }
    // every class reads the same x: only the first waits for the step before
    if (const int e = push(pj.bits, pj.group, x, m, k, c, wt, st, y, nn, ld, bf16w, !first || independent, false))
      return e;
    first = false;
  }
  return 0;
}

int LinearChain::build() {
  if (chain_ || steps_.empty()) return 1;
  return ak_wq_chain_create(steps_.data(), (int)steps_.size(), &chain_);
}

int LinearChain::run(void* stream) { return chain_ ? ak_wq_chain_run(chain_, stream) : 1; }

bool LinearChain::chained() const { return chain_ && ak_wq_chain_chained(chain_) == 1; }

}  // namespace agens
