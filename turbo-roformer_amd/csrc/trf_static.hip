// trf_stack_forward_static: the stack forward for callers that cannot allocate device memory.  Its
// workspace is a static device array in this file, one copy per GPU; host code reaches it only through
// the device address hipGetSymbolAddress returns for the current device, looked up once per device.
#include <mutex>

#include "trf_hip.h"
#include "trf_internal.h"

namespace {

// The workspace (xn, O, G and the Q/K/V^T sequence buffers of trf_stack_forward) of every call on a GPU.
// In host code this name is only a stand-in for the symbol, not a device address.
static __device__ __align__(256) uint8_t scratch[TRF_STATIC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once looked up

// This device's copy of `scratch`: looked up on the first call with the device current, then cached.
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return trf::set_error(TRF_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return trf::set_error(TRF_ERR_ARG, "device %d is out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return trf::set_error(TRF_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                            hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TRF_OK;
}

}  // namespace

extern "C" int trf_stack_forward_static(float* X, int32_t batch, int32_t T, int32_t F,
                                        const void* const* packed_layers, const int32_t* modes, int32_t n_layers,
                                        int32_t precision, const float* rope_time, const float* rope_freq,
                                        trf_stream_t stream) {
  const size_t need = trf_stack_workspace_bytes(batch, T, F);
  if (need == 0) return TRF_ERR_ARG;  // bad shape; the message is set
  if (need > TRF_STATIC_WORKSPACE_BYTES)
    return trf::set_error(TRF_ERR_WORKSPACE,
                          "batch %d x T %d x F %d needs %zu bytes of workspace; the static workspace holds %zu "
                          "(use trf_stack_forward with a caller-owned workspace)",
                          batch, T, F, need, size_t(TRF_STATIC_WORKSPACE_BYTES));
  void* ws = nullptr;
  if (int rc = scratch_on_current_device(&ws)) return rc;
  return trf_stack_forward(X, batch, T, F, packed_layers, modes, n_layers, precision, rope_time, rope_freq, ws,
                           TRF_STATIC_WORKSPACE_BYTES, stream);
}
