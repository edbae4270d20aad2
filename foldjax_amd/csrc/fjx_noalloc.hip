// fjx_trimul_fwd_noalloc: the triangle multiplicative update for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc). Its workspace is a static device
// array of this file, one copy per GPU, reserved when the library's code is
// loaded on that GPU and held until the process ends.
//
// The array's name is a host-side shadow: host code never passes it to a
// kernel or a copy. Its device address is obtained once per device with
// hipGetSymbolAddress, with that device current, and kept in g_scratch.
// Nothing in this path calls hipMalloc, hipFree or an allocating library
// routine, and no timing event is created.
#include <cstdio>
#include <mutex>

#include <hip/hip_runtime.h>

#include "fjx_tri.h"

static __device__ __align__(256) unsigned char scratch[FJX_NOALLOC_SCRATCH_BYTES];

namespace fjx {
int trimul_fwd_on_scratch(const fjx_trimul_args* a, hipStream_t st, void* scratch_ptr, size_t scratch_bytes,
                          const char* fn);
int set_error(int code, const char* msg);
}  // namespace fjx

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch` on each device, once resolved

// the address of this device's copy of `scratch`, resolved on first use with
// the device current; null (and an error message) on failure
void* scratch_on(int dev, char* err, size_t err_len) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_scratch[dev]) return g_scratch[dev];
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) {
    snprintf(err, err_len, "fjx_trimul_fwd_noalloc: hipGetSymbolAddress of the static scratch failed on device %d: %s",
             dev, hipGetErrorString(e));
    return nullptr;
  }
  g_scratch[dev] = ptr;
  return ptr;
}

}  // namespace

extern "C" int fjx_trimul_fwd_noalloc(const fjx_trimul_args* a, hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fjx::set_error(FJX_ERR_HIP, "fjx_trimul_fwd_noalloc: no current HIP device");
  if (stream) {
    // the kernels run on the stream's device; its copy of the scratch is the
    // one to use, so the stream must belong to the current device
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess)
      return fjx::set_error(FJX_ERR_HIP, "fjx_trimul_fwd_noalloc: cannot query the stream's device");
    if (sdev != dev)
      return fjx::set_error(FJX_ERR_INVALID,
                            "fjx_trimul_fwd_noalloc: the stream belongs to another device than the current one");
  }
  char err[256];
  void* ptr = scratch_on(dev, err, sizeof err);
  if (!ptr) return fjx::set_error(FJX_ERR_HIP, err);
  return fjx::trimul_fwd_on_scratch(a, stream, ptr, FJX_NOALLOC_SCRATCH_BYTES, "fjx_trimul_fwd_noalloc");
}
