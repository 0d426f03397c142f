// Runtime entry points of the C ABI: device memory, copies, synchronisation, error strings.
// reference: kernels/src/runtime.cu:25-44 (agens_kernels.h:17-30); same semantics on the HIP runtime.
#include <string.h>

#include "agens_kernels.h"
#include "wq_common.h"

extern "C" {

int ak_device_count(int* n) { return (int)hipGetDeviceCount(n); }
int ak_set_device(int dev) { return (int)hipSetDevice(dev); }

int ak_device_name(int dev, char* buf, int len) {
  if (!buf || len < 1) return AK_INVALID;
  hipDeviceProp_t p;
  const hipError_t e = hipGetDeviceProperties(&p, dev);
  if (e != hipSuccess) return (int)e;
  const char* name = p.name[0] ? p.name : p.gcnArchName;
  strncpy(buf, name, (size_t)len - 1);
  buf[len - 1] = 0;
  return 0;
}

int ak_malloc(void** ptr, size_t bytes) { return (int)hipMalloc(ptr, bytes); }
int ak_free(void* ptr) { return (int)hipFree(ptr); }
int ak_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}
int ak_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}
int ak_synchronize(void) { return (int)hipDeviceSynchronize(); }
int ak_mem_info(size_t* free_bytes, size_t* total_bytes) { return (int)hipMemGetInfo(free_bytes, total_bytes); }
const char* ak_error_string(int code) { return hipGetErrorString((hipError_t)code); }
// pinned, device-mapped host memory (the reference's cudaHostAlloc(Mapped)); allocated, never registered
int ak_host_alloc(void** ptr, size_t bytes) { return (int)hipHostMalloc(ptr, bytes, hipHostMallocMapped); }
int ak_host_free(void* ptr) { return (int)hipHostFree(ptr); }

}  // extern "C"
