// Host side of the quantized-linear path above the C ABI (include/agens_kernels.h), in C++.
//
// The reference's host code for this path is Rust (crates/agens-cuda/src/lib.rs: DeviceBuffer, upload,
// w4/w3/wq_upload_kt) and C++ (kernels/m1/m1_model.cu: W4Part / W4Lin, linear(), linear_shared()).  This mirrors their
// interface -- same names, argument meanings and error behaviour -- so the engine's load and decode code reads the
// same against this library.  Errors are thrown as agens::Error (the Rust side's anyhow::bail) where the reference
// bails, and returned as the reference's integer codes where it returns them (linear, linear_shared).
#pragma once
#include "agens_kernels.h"

#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace agens {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// check(): non-zero code -> "<what>: error <code> (<ak_error_string>)" (lib.rs:39-45)
void check(int code, const char* what);

// Owned device allocation (lib.rs DeviceBuffer, device_alloc, leak, Drop: lib.rs:225-262)
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t bytes);
  DeviceBuffer(DeviceBuffer&& o) noexcept;
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer();
  void* ptr() const { return ptr_; }
  size_t bytes() const { return bytes_; }
  void* leak();  // weights live for the process (lib.rs:229-234)

 private:
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
};

DeviceBuffer device_alloc(size_t bytes);
DeviceBuffer upload(const void* host, size_t bytes);  // device_alloc + H2D (lib.rs upload)

using KtPair = std::pair<DeviceBuffer, DeviceBuffer>;  // (wt, st): KT weights and scales

// int4-container linear [n, k] (packed: n*k/2 bytes, scales: n*k/group bf16) -> W4 KT (lib.rs w4_upload_kt)
KtPair w4_upload_kt(const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n, int k, int group);
// -> W3 KT, or nullopt when a value needs 4 bits (lib.rs w3_upload_kt:176-191)
std::optional<KtPair> w3_upload_kt(const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n,
                                   int k, int group);
// -> W{bits} KT; throws when a value needs more than `bits` bits (lib.rs wq_upload_kt:192-213)
KtPair wq_upload_kt(int bits, const std::vector<uint8_t>& packed, const std::vector<uint8_t>& scales, int n, int k,
                    int group);

// A quantized linear: one or two row parts (gate_up merged from parts of different bit width / group), part j writes
// rows [r0, r0 + n) of the output (m1_model.cu:121-132).
struct QuantPart {
  void *wt = nullptr, *st = nullptr;
  int r0 = 0, n = 0, group = 128, bits = 4;
};
struct QuantLinear {
  int n = 0, k = 0;
  int np = 0;
  QuantPart p[2];
};

// The model's linear (m1_model.cu:1857-1900): y[m][n] = x[m][k] W^T.  Up to 128 tokens one ak_wq_gemv_kt_multi per
// part with ldy = n; above, the prefill route (set_prefill_route): the fused GEMM ak_wq_gemm_kt per part, or tiles of
// output rows dequantized (ak_wq_dequant_kt_rows) into a bounded scratch of the process and multiplied by
// ak_bf16_linear_f32reduce(_ld).  Returns 0 or an error code; 1 for a shape
// mismatch.  The prefill route allocates its scratch on first use (not under stream capture) and is not re-entrant.
int linear(const QuantLinear& t, const void* x, void* y, int m, int n, int k, int bf16w, void* stream);
// bytes of one dequantized prefill tile (default 64 MB; the reference's tile bound, m1_model.cu:1822-1826)
void set_prefill_tile_bytes(size_t bytes);
// The prefill route above 128 tokens: -1 by shape (the default: the fused dequantize-in-GEMM kernel ak_wq_gemm_kt on
// every linear up to 256 tokens, long-k linears up to 1024 and wide linears up to 512 (LM-head-wide: 1024) tokens,
// where it was measured faster), 0 dequantized tiles x library
// GEMM (the reference's route), 1 the fused kernel.  Both give results within fp32-accumulation tolerance of the
// dequantized weights times x.
void set_prefill_route(int mode);

// Linears sharing x (m1_model.cu:1904-1937): one launch per (bits, group) class of single-part linears when m == 1
// (outputs bit-identical to separate GEMVs), otherwise one linear() each.
int linear_shared(const void* x, int nl, const QuantLinear* const* lins, void* const* ys, const int* ns, int m, int k,
                  int bf16w, void* stream);

// A run of consecutive GEMV calls of a decode step as one chained launch (ak_wq_chain_*): the role of the reference's
// captured decode graph whose GEMV kernels get programmatic-dependent-launch edges (runtime.cu:198-230 ak_graph_pdl,
// agens_pdl.cuh:1-16), so that each GEMV streams its weights while the one before it finishes.  Each call appended
// here is the linear() / linear_shared() call of the same arguments (same outputs, bit for bit); a step waits for the
// step before it unless declared independent (it reads nothing the step before writes).  Up to 128 tokens (the
// prefill route is not chained).  Not thread-safe; the buffers must stay valid while the chain is used.
class LinearChain {
 public:
  LinearChain() = default;
  LinearChain(const LinearChain&) = delete;
  LinearChain& operator=(const LinearChain&) = delete;
  ~LinearChain();
  // linear(t, x, y, m, t.n, t.k, bf16w): one step per part (a second part reads the same x: independent of the first).
  // act: x is the merged gate_up [m][2 * t.k] and the step's activations are SiLU(gate) * up (ak_wq_gemv_kt_silu;
  // single-part linears, default numerics).  1 for a bad argument or after build().
  int add(const QuantLinear& t, const void* x, void* y, int m, int bf16w = 0, bool independent = false,
          bool act = false);
  // linear_shared(x, nl, lins, ys, ns, m, k, bf16w): one step per (bits, group) class of the single-part linears (their
  // segments in one launch), a multi-part linear as add().  1 for a bad argument or after build().
  int add_shared(const void* x, int nl, const QuantLinear* const* lins, void* const* ys, const int* ns, int m, int k,
                 int bf16w = 0, bool independent = false);
  // ak_wq_chain_create over the steps: validates, allocates and uploads the step table (synchronous; not under stream
  // capture).  0 or an error code.
  int build();
  // one launch on `stream` (one launch per step where the chained kernels do not take a step: group 64, more than four
  // tokens, more than two with a fused activation step, exact numerics); allocates nothing and can be captured.  hipErrorNotReady (600) while the device's last
  // chained launch, issued on another stream, is still running (chained launches on one device share its flag words).
  int run(void* stream);
  // 1: runs as one chained launch, 0: as one launch per step (after build())
  bool chained() const;
  size_t steps() const { return steps_.size(); }

 private:
  int push(int bits, int group, const void* x, int m, int k, int nseg, const void* const* wt, const void* const* st,
           void* const* y, const int* n, const int* ldy, int bf16w, bool independent, bool act);
  std::vector<ak_wq_step> steps_;
  void* chain_ = nullptr;
};

}  // namespace agens
