// msda_internal.h — host <-> kernel parameter blocks and launcher declarations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "msda_device.h"

namespace msda {

constexpr int kMaxLevels = 64;

// Kernel parameters for one launch over a contiguous range of batches. Pointers are
// already offset to the first batch of the range; all in-kernel offsets are 32-bit.
struct Params {
  const void* value;       // (Bc, K, H, C) value_dtype
  const void* loc;         // (Bc, Q, H, L, P, dim) coord_dtype
  const void* attn;        // (Bc, Q, H, L, P) coord_dtype
  const void* grad_out;    // (Bc, Q, H*C) value_dtype (backward only)
  void* out;               // forward: (Bc, Q, H*C) value_dtype
  float* grad_acc;         // backward: fp32 (Bc, K, H, C) grad_value accumulator
  void* grad_loc;          // backward: like loc
  void* grad_attn;         // backward: like attn
  const int32_t* shapes;   // (L, dim)
  const int32_t* starts;   // (L,)
  uint32_t value_bytes;    // bytes of value in this launch (< 2^31)
  uint32_t acc_bytes;      // bytes of grad_acc in this launch (< 2^31)
  int32_t K, H, C, L, P;
  uint32_t Q;
  uint32_t num_units;      // Bc * Q * H
  FastDiv div_qh;          // divisor Q*H
  FastDiv div_qhg;         // divisor Q*HG (HG = 2^hg_log2 heads share a cache line)
  int32_t hg_log2;
  int32_t lpu_log2;        // lanes per unit = 2^lpu_log2 >= nvec
  int32_t nvec;            // C / VEC
  int32_t clamp;
  float lo_g, hi_g;        // grid clamp bounds as fp32
  uint32_t nblocks;
};

// dtype codes match msda_dtype in include/msda.h
using LaunchFn = hipError_t (*)(const Params&, hipStream_t);

// Returns the launcher for a (dim, value dtype, coord dtype, vector width) combination,
// or nullptr if it is not instantiated. vec_bytes is VEC * sizeof(value element).
LaunchFn get_fwd_launcher(int dim, int vdt, int cdt, int vec_bytes);
LaunchFn get_bwd_launcher(int dim, int vdt, int cdt, int vec_bytes);

hipError_t launch_fill_zero(float* p, size_t n, hipStream_t s);
hipError_t launch_narrow(const float* src, void* dst, int vdt, size_t n, hipStream_t s);

}  // namespace msda
