// Library-level state: thread-local error text and version string.
#include <stdarg.h>

#include "qh_common.h"

namespace qh {

static thread_local char g_err[1024] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace qh

extern "C" const char* qh_last_error(void) { return qh::g_err; }

extern "C" const char* qh_version(void) { return "qwen-hip 0.1.0 gfx950"; }

// Zero-fill kernel used instead of hipMemsetAsync so that callers may capture
// the library's launches into a HIP graph.
__global__ void qh_fill_zero_kernel(uint4* p, int64_t n16) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

__global__ void qh_fill_zero_bytes_kernel(unsigned char* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

extern "C" int qh_zero(void* ptr, int64_t nbytes, void* stream) {
  QH_CHECK_ARG(nbytes >= 0, "qh_zero: negative size");
  if (nbytes == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  if (aligned16(ptr) && nbytes % 16 == 0) {
    int64_t n16 = nbytes / 16;
    int64_t grid = ceil_div(n16, 256);
    if (grid > 4096) grid = 4096;
    qh_fill_zero_kernel<<<(int)grid, 256, 0, st>>>((uint4*)ptr, n16);
  } else {
    int64_t grid = ceil_div(nbytes, 256);
    if (grid > 4096) grid = 4096;
    qh_fill_zero_bytes_kernel<<<(int)grid, 256, 0, st>>>((unsigned char*)ptr, nbytes);
  }
  QH_CHECK_LAUNCH("qh_zero");
  return QH_OK;
}
