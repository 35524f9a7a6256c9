// msda_noalloc.hip — msda_bwd_noalloc: the backward with its workspace in a static device
// array instead of caller memory, for callers that cannot allocate device memory.
//
// The array is a file-scope __device__ object of MSDA_NOALLOC_SCRATCH_BYTES, so each GPU the
// library runs on holds its own copy from module load until the process ends. In host code
// its name is a host-side stand-in, never a device address: the entry point looks up each
// device's address once, with that device current, through hipGetSymbolAddress, and only
// ever hands that address to the kernels. Every call on one GPU shares that GPU's array
// (nothing in it has to start at zero: the backward writes every workspace word before it
// reads it, and clears its atomic sums with a kernel), so calls that overlap on one GPU, on
// different streams or threads, race.
#include <mutex>

#include "../../include/msda.h"
#include "msda_internal.h"

namespace {

constexpr size_t kScratchBytes = MSDA_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices];  // each device's address of `scratch`, once looked up

// The current device's address of `scratch`, looked up on the first call on that device.
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return msda::set_error(MSDA_ERR_HIP, "msda_bwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return msda::set_error(MSDA_ERR_INVALID, "msda_bwd_noalloc: device %d is beyond the %d supported",
                           dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return msda::set_error(MSDA_ERR_HIP, "msda_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                             dev, hipGetErrorString(e));
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return MSDA_OK;
}

}  // namespace

extern "C" {

int msda_bwd_noalloc(const msda_desc* d, const int32_t* host_spatial_shapes, const void* value,
                     const void* sampling_locations, const void* attention_weights,
                     const void* grad_output, void* grad_value, void* grad_sampling_locations,
                     void* grad_attention_weights, void* stream) {
  int rc = msda_validate(d);
  if (rc) return rc;
  const size_t need = msda_bwd_workspace_bytes(d, host_spatial_shapes);  // host only
  void* ws = nullptr;
  if (need > kScratchBytes)
    return msda::set_error(MSDA_ERR_WORKSPACE,
                           "msda_bwd_noalloc: this problem needs %zu bytes of backward workspace, "
                           "more than the static scratch of %zu bytes; call msda_bwd with a "
                           "caller workspace instead",
                           need, kScratchBytes);
  if (need > 0 && (rc = scratch_ptr(&ws))) return rc;
  // need == 0: nothing to sample, or invalid shapes, which msda_bwd reports before any launch
  return msda_bwd(d, host_spatial_shapes, value, sampling_locations, attention_weights,
                  grad_output, grad_value, grad_sampling_locations, grad_attention_weights, ws,
                  need, stream);
}

}  // extern "C"
