// lbmoe_forward_static: the whole block with its workspace in a library-owned device array, for
// callers that cannot allocate device memory. No counterpart in the reference.
//
// `scratch` is a file-scope device array of LBMOE_STATIC_WORKSPACE_BYTES; every GPU the library
// runs on holds its own copy until the process ends. In host code its name is only a stand-in
// for the device address, so the address is looked up once per device with
// hipGetSymbolAddress (with that device current) and kept; kernels get that address, never the
// array's name. The block's kernels clear what they count in (counters, histograms, the tile
// list) themselves and write every other region before reading it, so nothing in the array has
// to start at zero and the previous call's contents do no harm. Calls that overlap on one GPU
// (two streams, or two host threads) share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.hpp"

namespace lbmoe {

static __device__ __align__(256) unsigned char scratch[LBMOE_STATIC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch[kMaxDevices];   // device address of `scratch`, per device (null: unknown)
static std::mutex g_scratch_mu;

// Address of the current device's `scratch`, looked up on the first call on that device.
static int32_t scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return LBMOE_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    // The first call may come while the caller's stream is being captured into a graph: the
    // lookup is not stream work, so this thread's capture mode is relaxed around it (a capture
    // in the global or thread-local mode would otherwise refuse a runtime call that may load
    // the code object) and restored afterwards.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return LBMOE_ERR_DEVICE;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return LBMOE_ERR_DEVICE;
    if (e != hipSuccess || !p) return LBMOE_ERR_DEVICE;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return LBMOE_OK;
}

}  // namespace lbmoe

extern "C" int32_t lbmoe_forward_static(const lbmoe_layer* layer, const void* x, int64_t T,
                                        void* y, void* stream) {
  size_t need = 0;
  int32_t st = lbmoe_workspace_size(layer, T, &need);
  if (st != LBMOE_OK) return st;
  if (need > LBMOE_STATIC_WORKSPACE_BYTES) return LBMOE_ERR_STATIC_LIMIT;
  if (T == 0) return lbmoe_forward(layer, x, T, y, nullptr, 0, stream);
  void* ws = nullptr;
  if ((st = lbmoe::scratch_of_current_device(&ws)) != LBMOE_OK) return st;
  return lbmoe_forward(layer, x, T, y, ws, LBMOE_STATIC_WORKSPACE_BYTES, stream);
}
