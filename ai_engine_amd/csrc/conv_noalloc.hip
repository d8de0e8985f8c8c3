// conv_noalloc.hip -- aih_conv_noalloc: aih_conv for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). The only device memory aih_conv needs
// beyond its inputs and outputs is the split-K workspace (fp32 partial sums,
// [split][M][N4]); here it is a fixed array in the library's own device
// segment instead of a caller buffer.
//
// The array is one per device, set up the first time a device calls in
// (hipGetSymbolAddress with that device current), and held until the process
// ends. Every call on a device shares it, so calls that overlap on one device
// (different streams, or host threads without ordering) race on it; calls
// ordered on one stream do not. The split-K kernels overwrite every partial
// they later read, so nothing in it has to start at zero and the previous
// call's contents never leak into a result.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/aih_conv.h"
#include "capi_util.h"

constexpr size_t kScratchBytes = AIH_NOALLOC_SCRATCH_BYTES;

// The workspace of aih_conv_noalloc. In host code `scratch` names a host-side
// stand-in, not device memory: only the address from hipGetSymbolAddress may
// reach a kernel.
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;

// Device address of this device's copy of `scratch`, or null with the
// reason in *why.
void *scratch_of_current_device(std::string *why) {
  static std::mutex mu;
  static void *ptrs[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *why = std::string("no current device: ") + hipGetErrorString(e);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      *why = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace

extern "C" {

int aih_conv_noalloc(const aih_conv_desc *d, const void *x, const void *w, const void *bias, const void *res,
                     void *y, aih_stream stream) {
  return aih::api_guarded([&] {
    if (aih_conv_check(d)) return AIH_ERR;
    const size_t need = aih_conv_workspace_size(d);
    if (need > kScratchBytes)
      return aih::api_fail("conv_noalloc: this conv needs " + std::to_string(need) +
                           " bytes of split-K workspace, above the " + std::to_string(kScratchBytes) +
                           "-byte scratch; call aih_conv with a workspace");
    void *ws = nullptr;
    if (need) {
      std::string why;
      ws = scratch_of_current_device(&why);
      if (!ws) return aih::api_fail("conv_noalloc: " + why);
    }
    return aih_conv(d, x, w, bias, res, y, ws, need ? kScratchBytes : 0, stream);
  });
}

}  // extern "C"
