// Library-level plumbing: thread-local error text, launch checks, pinned host pool memory.
#include <cstring>

#include "omm_common.h"

namespace omm {

namespace {
thread_local char g_err[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(OMM_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return OMM_OK;
}

namespace {
__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = value;
}
}  // namespace

int fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t stream) {
  if (n <= 0) return OMM_OK;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv64(n, 256), 4096));
  fill_i32_kernel<<<blocks, 256, 0, stream>>>(p, n, value);
  return check_launch("fill");
}

}  // namespace omm

extern "C" {

const char* omm_last_error(void) { return omm::g_err; }

int omm_abi_version(void) { return 4; }

int omm_host_alloc(size_t bytes, void** host, void** dev) {
  OMM_REQUIRE(host != nullptr && dev != nullptr, OMM_EINVAL, "omm_host_alloc: null output");
  *host = nullptr;
  *dev = nullptr;
  if (bytes == 0) return OMM_OK;
  void* h = nullptr;
  hipError_t e = hipHostMalloc(&h, bytes, hipHostMallocMapped | hipHostMallocPortable);
  if (e != hipSuccess)
    return omm::set_error(OMM_EHIP, "omm_host_alloc(%zu): %s", bytes, hipGetErrorString(e));
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, h, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(h);
    return omm::set_error(OMM_EHIP, "omm_host_alloc: device pointer: %s", hipGetErrorString(e));
  }
  *host = h;
  *dev = d;
  return OMM_OK;
}

int omm_host_free(void* host) {
  if (host == nullptr) return OMM_OK;
  const hipError_t e = hipHostFree(host);
  if (e != hipSuccess) return omm::set_error(OMM_EHIP, "omm_host_free: %s", hipGetErrorString(e));
  return OMM_OK;
}

}  // extern "C"
