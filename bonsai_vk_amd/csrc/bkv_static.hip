// bkv_static.hip - bkv_decode_step_static: bkv_decode_step with its workspace in a static device
// array instead of a caller buffer, for callers that cannot allocate (code under graph capture,
// serving loops that forbid hipMalloc). Nothing here allocates: the array is part of the loaded
// code object, one copy per GPU, held until the process ends.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/bkv.h"
#include "bkv_internal.h"

namespace bkv {

// the workspace of every bkv_decode_step_static call on one GPU (zeroed once, on that GPU's first
// call). 16 MiB holds the decode plan of about 64K keys at nkv = 4.
constexpr size_t kStaticScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// per device: the array's device address (the host-side name `scratch` is not one)
constexpr int kMaxDevices = 64;
static void *g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

// the device address of the current device's array, zeroed by a fill kernel on `stream` the first
// time (stream-ordered before this call's kernels); nullptr and the HIP error on failure
static void *device_scratch(hipStream_t stream, hipError_t *err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *ptr = nullptr;
    *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    *err = launch_workspace_init(static_cast<unsigned *>(ptr), kStaticScratchBytes / sizeof(unsigned), stream);
    if (*err != hipSuccess) return nullptr;
    g_scratch[dev] = ptr;
  }
  return g_scratch[dev];
}

}  // namespace bkv

using namespace bkv;

extern "C" {

size_t bkv_static_scratch_bytes(void) { return kStaticScratchBytes; }

int bkv_decode_step_static(const bkv_cache_desc *d, int layer, uint32_t pos, const float *k,
                           const float *v, const float *q, const float *gate, float *out,
                           float *out_gated, hipStream_t stream) {
  int rc = bkv_geom_check(d);
  if (rc) return rc;
  // the decode plan of pos + 1 keys must fit the array (bkv_decode_step reports every other error)
  if (pos == 0xFFFFFFFFu) return BKV_ECAP;
  uint64_t lay[6];
  if ((rc = bkv_debug_layout(d, pos + 1, lay))) return rc;
  if (lay[5] > kStaticScratchBytes) return BKV_ESCRATCH;
  hipError_t e = hipSuccess;
  void *ws = device_scratch(stream, &e);
  if (!ws) return hip_fail(e);
  return bkv_decode_step(d, layer, pos, k, v, q, gate, out, out_gated, ws, kStaticScratchBytes, stream);
}

int bkv_static_error(const bkv_cache_desc *d, hipStream_t stream) {
  int rc = bkv_geom_check(d);
  if (rc) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e);
  if (dev < 0 || dev >= kMaxDevices) return hip_fail(hipErrorInvalidDevice);
  void *ws = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ws = g_scratch[dev];
  }
  if (!ws) return BKV_OK;                       // no static call has run on this device
  // bkv_workspace_error on the array: it synchronises the stream, reads the error word and, when
  // it is set, zeroes the whole array (the workspace of every later static call on this device)
  return bkv_workspace_error(d, ws, kStaticScratchBytes, stream);
}

int bkv_static_debug_address(void **out) {
  if (!out) return BKV_EINVAL;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e);
  if (dev < 0 || dev >= kMaxDevices) return hip_fail(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  *out = g_scratch[dev];
  return BKV_OK;
}

int bkv_static_reset(hipStream_t stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e);
  if (dev < 0 || dev >= kMaxDevices) return hip_fail(hipErrorInvalidDevice);
  void *ws = device_scratch(stream, &e);
  if (!ws) return hip_fail(e);
  return hip_fail(launch_workspace_init(static_cast<unsigned *>(ws), kStaticScratchBytes / sizeof(unsigned), stream));
}

}  // extern "C"
