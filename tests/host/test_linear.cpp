// GPU test of the C++ host side (agens-engine_amd/host/agens_linear.h): uploads, linear() and linear_shared() against
// direct C-ABI launches, bit for bit, plus the error behaviour of the reference's host code (lib.rs:176-213,
// m1_model.cu:1857-1937).  Run by tests/test_host_linear.py; prints "host linear: OK" on success.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "agens_kernels.h"
#include "agens_linear.h"

using namespace agens;

static uint32_t g_state = 2463534242u;
static uint32_t rnd() {
  g_state ^= g_state << 13, g_state ^= g_state >> 17, g_state ^= g_state << 5;
  return g_state;
}
static uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1)) >> 16);
}
static int fails = 0;
#define EXPECT(c, what)                                   \
  do {                                                    \
    if (!(c)) {                                           \
      std::fprintf(stderr, "FAILED: %s (%s)\n", what, #c); \
      ++fails;                                            \
    }                                                     \
  } while (0)

// int4 container [n, k] with codes of `bits` bits, and bf16 scales
static void container(int n, int k, int group, int bits, std::vector<uint8_t>& packed, std::vector<uint8_t>& scales) {
  const int lo = -(1 << (bits - 1)), span = 1 << bits;
  packed.assign((size_t)n * k / 2, 0);
  for (size_t i = 0; i < packed.size(); ++i) {
    const int q0 = lo + (int)(rnd() % span), q1 = lo + (int)(rnd() % span);
    packed[i] = (uint8_t)((q0 + 8) | ((q1 + 8) << 4));
  }
  scales.resize((size_t)n * (k / group) * 2);
  for (size_t i = 0; i < scales.size(); i += 2) {
    const uint16_t s = f2bf(0.002f + 0.03f * (rnd() >> 8) / 16777216.f);
    std::memcpy(&scales[i], &s, 2);
  }
}
static std::vector<uint16_t> get(const void* d, size_t n) {
  std::vector<uint16_t> h(n);
  check(ak_synchronize(), "sync");
  check(ak_memcpy_d2h(h.data(), d, n * 2), "d2h");
  return h;
}

int main() {
  int ndev = 0;
  check(ak_device_count(&ndev), "device_count");
  if (ndev < 1) {
    std::printf("no GPU\n");
    return 1;
  }
  const int k = 1024, g = 128;
  // ---- a gate_up-style linear of two parts with different bit widths (W3 rows 0..95, W4 rows 96..159)
  std::vector<uint8_t> p0, s0, p1, s1;
  container(96, k, g, 3, p0, s0);
  container(64, k, g, 4, p1, s1);
  KtPair a = wq_upload_kt(3, p0, s0, 96, k, g), b = wq_upload_kt(4, p1, s1, 64, k, g);
  QuantLinear gu;
  gu.n = 160, gu.k = k, gu.np = 2;
  gu.p[0] = {a.first.ptr(), a.second.ptr(), 0, 96, g, 3};
  gu.p[1] = {b.first.ptr(), b.second.ptr(), 96, 64, g, 4};
  for (int m : {1, 4}) {
    std::vector<uint16_t> hx((size_t)m * k);
    for (auto& v : hx) v = f2bf(-1.f + 2.f * (rnd() >> 8) / 16777216.f);
    DeviceBuffer x = upload(hx.data(), hx.size() * 2), y(m * 160 * 2), y0(m * 96 * 2), y1(m * 64 * 2);
    EXPECT(linear(gu, x.ptr(), y.ptr(), m, 160, k, 0, nullptr) == 0, "linear");
    const void* w0 = a.first.ptr();
    const void* t0 = a.second.ptr();
    const void* w1 = b.first.ptr();
    const void* t1 = b.second.ptr();
    void* q0 = y0.ptr();
    void* q1 = y1.ptr();
    const int n0 = 96, n1 = 64;
    check(ak_wq_gemv_kt_multi(3, x.ptr(), m, 1, &w0, &t0, &q0, &n0, nullptr, k, g, 0, nullptr), "direct W3");
    check(ak_wq_gemv_kt_multi(4, x.ptr(), m, 1, &w1, &t1, &q1, &n1, nullptr, k, g, 0, nullptr), "direct W4");
    const auto hy = get(y.ptr(), (size_t)m * 160), h0 = get(y0.ptr(), (size_t)m * 96), h1 = get(y1.ptr(), (size_t)m * 64);
    bool same = true;
    for (int j = 0; j < m; ++j)
      for (int r = 0; r < 160; ++r)
        same = same && hy[(size_t)j * 160 + r] == (r < 96 ? h0[(size_t)j * 96 + r] : h1[(size_t)j * 64 + r - 96]);
    EXPECT(same, "linear parts == direct launches");
    EXPECT(linear(gu, x.ptr(), y.ptr(), m, 161, k, 0, nullptr) == 1, "shape mismatch -> 1");
  }
  // ---- prefill (m > 128): dequantized tiles x GEMM, against fp64 products of the dequantized weights (tolerance of an
  // fp32-accumulated GEMM: 1 bf16 ulp of the result + 1e-5 of sum |x * w|), one tile and tiles of 256 rows
  {
    const int m = 200, n = 160;
    std::vector<uint16_t> hx((size_t)m * k);
    for (auto& v : hx) v = f2bf(-1.f + 2.f * (rnd() >> 8) / 16777216.f);
    DeviceBuffer x = upload(hx.data(), hx.size() * 2), y((size_t)m * n * 2), wd((size_t)n * k * 2);
    check(ak_wq_dequant_kt_rows(3, a.first.ptr(), a.second.ptr(), wd.ptr(), 96, k, g, 0, 96, nullptr), "dequant W3");
    check(ak_wq_dequant_kt_rows(4, b.first.ptr(), b.second.ptr(), static_cast<uint16_t*>(wd.ptr()) + (size_t)96 * k, 64,
                                k, g, 0, 64, nullptr),
          "dequant W4");
    const auto hw = get(wd.ptr(), (size_t)n * k);
    auto bf = [](uint16_t b) {
      uint32_t u = (uint32_t)b << 16;
      float f;
      std::memcpy(&f, &u, 4);
      return (double)f;
    };
    // routes: dequantized tiles (one tile, tiles of 256 rows) x library GEMM, then the fused GEMM (two parts of
    // different bits into one output)
    for (int route = 0; route < 3; ++route) {
      set_prefill_route(route < 2 ? 0 : 1);
      set_prefill_tile_bytes(route == 1 ? (size_t)256 * k * 2 : (size_t)64 << 20);
      EXPECT(linear(gu, x.ptr(), y.ptr(), m, n, k, 0, nullptr) == 0, "prefill linear");
      const auto hy = get(y.ptr(), (size_t)m * n);
      int bad = 0;
      for (int i = 0; i < m; ++i)
        for (int r = 0; r < n; ++r) {
          double ref = 0, mag = 0;
          for (int c = 0; c < k; ++c) {
            const double p = bf(hx[(size_t)i * k + c]) * bf(hw[(size_t)r * k + c]);
            ref += p, mag += std::fabs(p);
          }
          const double ulp = std::ldexp(1.0, (int)std::floor(std::log2(std::fabs(ref) + 1e-30)) - 7);
          bad += std::fabs(bf(hy[(size_t)i * n + r]) - ref) > ulp + 1e-5 * mag;
        }
      EXPECT(bad == 0, "prefill linear == dequantized weights x x");
    }
    set_prefill_tile_bytes((size_t)64 << 20);
    set_prefill_route(-1);
  }
  // ---- linear_shared: three single-part linears of mixed bits sharing x (two classes: W3 and W4)
  std::vector<uint8_t> pa, sa, pb, sb, pc, sc;
  container(64, k, g, 3, pa, sa);
  container(32, k, g, 4, pb, sb);
  container(48, k, g, 3, pc, sc);
  KtPair la = wq_upload_kt(3, pa, sa, 64, k, g), lb = wq_upload_kt(4, pb, sb, 32, k, g),
         lc = wq_upload_kt(3, pc, sc, 48, k, g);
  QuantLinear A, B, C;
  A.n = 64, B.n = 32, C.n = 48;
  A.k = B.k = C.k = k;
  A.np = B.np = C.np = 1;
  A.p[0] = {la.first.ptr(), la.second.ptr(), 0, 64, g, 3};
  B.p[0] = {lb.first.ptr(), lb.second.ptr(), 0, 32, g, 4};
  C.p[0] = {lc.first.ptr(), lc.second.ptr(), 0, 48, g, 3};
  std::vector<uint16_t> hx(k);
  for (auto& v : hx) v = f2bf(-1.f + 2.f * (rnd() >> 8) / 16777216.f);
  DeviceBuffer x = upload(hx.data(), hx.size() * 2);
  DeviceBuffer ya(128), yb(64), yc(96), ra(128), rb(64), rc(96);
  const QuantLinear* lins[3] = {&A, &B, &C};
  void* ys[3] = {ya.ptr(), yb.ptr(), yc.ptr()};
  const int ns[3] = {64, 32, 48};
  EXPECT(linear_shared(x.ptr(), 3, lins, ys, ns, 1, k, 0, nullptr) == 0, "linear_shared");
  EXPECT(linear(A, x.ptr(), ra.ptr(), 1, 64, k, 0, nullptr) == 0, "linear A");
  EXPECT(linear(B, x.ptr(), rb.ptr(), 1, 32, k, 0, nullptr) == 0, "linear B");
  EXPECT(linear(C, x.ptr(), rc.ptr(), 1, 48, k, 0, nullptr) == 0, "linear C");
  EXPECT(get(ya.ptr(), 64) == get(ra.ptr(), 64), "shared A == separate");
  EXPECT(get(yb.ptr(), 32) == get(rb.ptr(), 32), "shared B == separate");
  EXPECT(get(yc.ptr(), 48) == get(rc.ptr(), 48), "shared C == separate");
  // ---- LinearChain: two decoder layers (qkv of mixed bits through add_shared, o, a two-part gate_up W3 | W2, down
  // with the SiLU(gate) * up activation) as one chained launch, equal bit for bit to the same calls one at a time
  // (linear_shared, linear, ak_wq_gemv_kt_silu); 1 and 2 tokens chained, 4 tokens one launch per step
  {
    const int H = 1024, KV = 256, I = 16384;  // the fused activation is chained on split-K down steps (k >= 16384)
    struct Layer {
      std::vector<KtPair> kt;
      QuantLinear q, kk, v, o, gu, dn;
    };
    auto make_lin = [&](Layer& L, QuantLinear& t, int n, int kin, int bits) {
      std::vector<uint8_t> p, sc;
      container(n, kin, g, bits, p, sc);
      L.kt.push_back(wq_upload_kt(bits, p, sc, n, kin, g));
      t.n = n, t.k = kin, t.np = 1;
      t.p[0] = {L.kt.back().first.ptr(), L.kt.back().second.ptr(), 0, n, g, bits};
    };
    Layer layers[2];
    for (int li = 0; li < 2; ++li) {
      Layer& L = layers[li];
      L.kt.reserve(8);
      make_lin(L, L.q, H, H, 3);
      make_lin(L, L.kk, KV, H, 3);
      make_lin(L, L.v, KV, H, 4);
      make_lin(L, L.o, H, H, 4);
      QuantLinear gate, up;
      make_lin(L, gate, I, H, 3);
      make_lin(L, up, I, H, 2);
      L.gu.n = 2 * I, L.gu.k = H, L.gu.np = 2;
      L.gu.p[0] = gate.p[0];
      L.gu.p[1] = up.p[0];
      L.gu.p[1].r0 = I;
      make_lin(L, L.dn, H, I, li ? 2 : 3);
    }
    for (int m : {1, 2, 4}) {
      std::vector<uint16_t> hh((size_t)m * H);
      for (auto& v : hh) v = f2bf(-1.f + 2.f * (rnd() >> 8) / 16777216.f);
      DeviceBuffer h = upload(hh.data(), hh.size() * 2);
      // outputs: [run][layer] q, k, v, o, gate_up, down
      std::vector<DeviceBuffer> out[2][2];
      for (int r = 0; r < 2; ++r)
        for (int li = 0; li < 2; ++li) {
          for (int n : {H, KV, KV, H, 2 * I, H}) out[r][li].emplace_back((size_t)m * n * 2);
        }
      LinearChain ch;
      const void* x = h.ptr();
      for (int li = 0; li < 2; ++li) {
        Layer& L = layers[li];
        auto& o = out[0][li];
        const QuantLinear* lins[3] = {&L.q, &L.kk, &L.v};
        void* ys[3] = {o[0].ptr(), o[1].ptr(), o[2].ptr()};
        const int ns[3] = {H, KV, KV};
        EXPECT(ch.add_shared(x, 3, lins, ys, ns, m, H) == 0, "chain add_shared");
        EXPECT(ch.add(L.o, o[0].ptr(), o[3].ptr(), m) == 0, "chain add o");
        EXPECT(ch.add(L.gu, o[3].ptr(), o[4].ptr(), m) == 0, "chain add gate_up");
        EXPECT(ch.add(L.dn, o[4].ptr(), o[5].ptr(), m, 0, false, true) == 0, "chain add down");
        x = o[5].ptr();
      }
      EXPECT(ch.build() == 0, "chain build");
      EXPECT(ch.chained() == (m <= 2), "chained for 1 and 2 tokens (a fused activation step: chained up to 2)");
      EXPECT(ch.add(layers[0].o, h.ptr(), out[0][0][3].ptr(), m) == 1, "add after build -> 1");
      EXPECT(ch.run(nullptr) == 0, "chain run");
      check(ak_synchronize(), "sync");
      EXPECT(ak_wq_chain_status() == 0, "chain status");
      // the same calls one at a time
      x = h.ptr();
      for (int li = 0; li < 2; ++li) {
        Layer& L = layers[li];
        auto& o = out[1][li];
        const QuantLinear* lins[3] = {&L.q, &L.kk, &L.v};
        void* ys[3] = {o[0].ptr(), o[1].ptr(), o[2].ptr()};
        const int ns[3] = {H, KV, KV};
        EXPECT(linear_shared(x, 3, lins, ys, ns, m, H, 0, nullptr) == 0, "linear_shared");
        EXPECT(linear(L.o, o[0].ptr(), o[3].ptr(), m, H, H, 0, nullptr) == 0, "linear o");
        EXPECT(linear(L.gu, o[3].ptr(), o[4].ptr(), m, 2 * I, H, 0, nullptr) == 0, "linear gate_up");
        const QuantPart& d = L.dn.p[0];
        EXPECT(ak_wq_gemv_kt_silu(d.bits, o[4].ptr(), m, d.wt, d.st, o[5].ptr(), H, 0, I, g, nullptr) == 0,
               "silu gemv");
        x = o[5].ptr();
      }
      bool same = true;
      for (int li = 0; li < 2; ++li)
        for (size_t i = 0; i < out[0][li].size(); ++i) {
          const size_t cnt = out[0][li][i].bytes() / 2;
          same = same && get(out[0][li][i].ptr(), cnt) == get(out[1][li][i].ptr(), cnt);
        }
      EXPECT(same, "chained steps == one call at a time");
      // a second run on the same stream is ordered after the first: accepted
      EXPECT(ch.run(nullptr) == 0, "second chain run");
      check(ak_synchronize(), "sync");
    }
  }
  // ---- upload errors (lib.rs: size mismatch bails, W3 returns None on a 4-bit value, wq bails)
  std::vector<uint8_t> p4, s4;
  container(32, k, g, 4, p4, s4);
  p4[0] = 0x0F;  // codes -8 and 7: outside 3 and 2 bits
  EXPECT(!w3_upload_kt(p4, s4, 32, k, g).has_value(), "w3_upload_kt -> nullopt");
  bool threw = false;
  try {
    wq_upload_kt(2, p4, s4, 32, k, g);
  } catch (const Error&) {
    threw = true;
  }
  EXPECT(threw, "wq_upload_kt out of range -> Error");
  threw = false;
  try {
    wq_upload_kt(4, p4, s4, 33, k, g);
  } catch (const Error&) {
    threw = true;
  }
  EXPECT(threw, "size mismatch -> Error");
  if (fails) {
    std::printf("host linear: %d FAILED\n", fails);
    return 1;
  }
  std::printf("host linear: OK\n");
  return 0;
}
