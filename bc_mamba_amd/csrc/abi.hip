// Library-level entry points: version, error string, zero fill.
#include "bcm_common.hpp"

#include <string.h>

namespace bcm {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* fn) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(BCM_EHIP, "%s: HIP error: %s", fn, hipGetErrorString(e));
  return BCM_OK;
}

// Grid-stride zero fill: 16-byte stores on the aligned body, bytes at the
// unaligned head and tail.
__global__ __launch_bounds__(256) void k_zero(uint8_t* p, int64_t head, int64_t n16, int64_t tail) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (tid < head) p[tid] = 0;
  uint4* body = reinterpret_cast<uint4*>(p + head);
  for (int64_t i = tid; i < n16; i += stride) body[i] = make_uint4(0, 0, 0, 0);
  if (tid < tail) p[head + n16 * 16 + tid] = 0;
}

int zero_bytes(void* ptr, int64_t bytes, hipStream_t s, const char* fn) {
  if (bytes <= 0) return BCM_OK;
  if (!ptr) return set_error(BCM_EINVAL, "%s: null pointer", fn);
  const uintptr_t a = reinterpret_cast<uintptr_t>(ptr);
  int64_t head = (int64_t)((16 - (a & 15)) & 15);
  if (head > bytes) head = bytes;
  const int64_t n16 = (bytes - head) / 16;
  const int64_t tail = bytes - head - n16 * 16;
  int64_t blocks = (n16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(k_zero, dim3((unsigned)blocks), dim3(256), 0, s, (uint8_t*)ptr, head, n16, tail);
  return check_launch(fn);
}

}  // namespace bcm

extern "C" {

int bcm_abi_version(void) { return BCM_ABI_VERSION; }

const char* bcm_last_error(void) { return bcm::g_err; }

int64_t bcm_bitmask_words(int64_t L) { return L <= 0 ? 0 : bcm::bitmask_words(L); }

int64_t bcm_tile_count(int64_t L) { return L <= 0 ? 0 : bcm::tile_count(L); }

int bcm_zero(void* ptr, int64_t bytes, bcm_stream_t stream) {
  return bcm::zero_bytes(ptr, bytes, bcm::hs(stream), "bcm_zero");
}

}  // extern "C"
