// Host side of the quantized-linear path above the C ABI (include/agens_kernels.h), in C++.
//
// The reference's host code for this path is Rust (crates/agens-cuda/src/lib.rs: DeviceBuffer, upload,
// w4/w3/wq_upload_kt) and C++ (kernels/m1/m1_model.cu: W4Part / W4Lin, linear(), linear_shared()).  This mirrors their
// interface -- same names, argument meanings and error behaviour -- so the engine's load and decode code reads the
// same against this library.  Errors are thrown as agens::Error (the Rust side's anyhow::bail) where the reference
// bails, and returned as the reference's integer codes where it returns them (linear, linear_shared).
#pragma once
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
// long-k linears, and on wide linears up to 384 tokens, where it was measured faster), 0 dequantized tiles x library
// GEMM (the reference's route), 1 the fused kernel.  Both give results within fp32-accumulation tolerance of the
// dequantized weights times x.
void set_prefill_route(int mode);

// Linears sharing x (m1_model.cu:1904-1937): one launch per (bits, group) class of single-part linears when m == 1
// (outputs bit-identical to separate GEMVs), otherwise one linear() each.
int linear_shared(const void* x, int nl, const QuantLinear* const* lins, void* const* ys, const int* ns, int m, int k,
                  int bf16w, void* stream);

}  // namespace agens
