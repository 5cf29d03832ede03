// lwl_bfht_backward_noalloc: the latent-gradient backward of lwl_bfht_backward
// with its scratch (one partial row per overlapped block, or the float32 work
// buffer of the multi-pass blocks) taken from a file-scope device array instead
// of a caller-provided workspace, for callers that cannot allocate (code under
// HIP graph capture, tight serving loops).
//
// The array is a per-device symbol: each GPU the library runs on holds its own
// copy, at its own address, until the process ends.  Host code never passes the
// symbol's name to a kernel (on the host it is only a stand-in); the device
// address comes from hipGetSymbolAddress, called once per device with that
// device current, and is cached per device.  Every call on one GPU shares that
// GPU's array: calls that overlap on one GPU (two streams, two threads) race on
// it.  The backward kernels write every scratch element they later read (each
// block's row over [0, latent_size), or the whole work buffer in the first
// pass), so nothing needs clearing between calls.
#include "../../include/lwl_bfht.h"

#include <hip/hip_runtime.h>

#include <atomic>

#include "bfht_launch.h"

namespace lwl {

static __device__ __align__(256) unsigned char scratch[LWL_BFHT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

}  // namespace

// Device address of `scratch` on the device that stream `s` belongs to (the
// current device for the null stream), or nullptr with the HIP error in *err.
// The first use on a device makes that device current for hipGetSymbolAddress
// (the address is per device) and restores the caller's device after it.
void* noalloc_scratch(hipStream_t s, hipError_t* err) {
  int cur = -1;
  *err = hipGetDevice(&cur);
  if (*err != hipSuccess) return nullptr;
  int dev = cur;
  if (s != nullptr) {
    hipDevice_t d = 0;
    *err = hipStreamGetDevice(s, &d);
    if (*err != hipSuccess) return nullptr;
    dev = (int)d;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  if (dev != cur && (*err = hipSetDevice(dev)) != hipSuccess) return nullptr;
  *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (dev != cur) {
    const hipError_t e2 = hipSetDevice(cur);
    if (*err == hipSuccess) *err = e2;
  }
  if (*err != hipSuccess || !p) {
    if (*err == hipSuccess) *err = hipErrorInvalidSymbol;
    return nullptr;
  }
  g_scratch_ptr[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace lwl
