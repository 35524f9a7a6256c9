// msda_fused.hip — producer-side kernels around the backward of the fused forward.
//
// The fused forward forms, per unit (b, q, h), in fp32:
//   loc[b,q,h,l,p,d] = fma(off[b,q,h,l,p,d], inv_l[d], ref[b,q,l,d]),
//                      inv_l = (1/W_l, 1/H_l[, 1/D_l]) rounded to fp32
//   attn[b,q,h,l,p]  = exp(logit - max) * (1 / sum exp(logit - max)) over (l, p)
// which is the location and weight formation of the reference modules
// (src/msda_triton/pytorch/msda_2d.py:303-339, msda_3d.py:314-350) done inside the kernel.
// Its backward runs the ordinary backward kernels on fp32 loc/attn written by
// fused_prep_kernel, then fused_grad_kernel takes grad_loc / grad_attn through that
// formation:
//   grad_off    = grad_loc * inv_l
//   grad_ref    = sum over (h, p) of grad_loc
//   grad_logits = attn * (grad_attn - sum over (l, p) of attn * grad_attn)
// Every output element is written once by one thread, in a fixed order of additions. The
// locations are bit-identical to the forward's (same fma, same reciprocals); the weights
// agree to rounding (the forward reduces the sum over its lanes, this kernel in order).
#include "msda_internal.h"
#include "msda_sample.h"

namespace msda {

namespace {

template <typename E>
__device__ inline float ld(const void* p, uint32_t i) {
  return (float)static_cast<const typename E::T*>(p)[i];
}

template <typename E>
__device__ inline void st(void* p, uint32_t i, float v) {
  static_cast<typename E::T*>(p)[i] = (typename E::T)v;
}

// Indices are 32-bit: one launch covers a batch range whose units * L * P * 2^dim < 2^31.

// Unit u's L*P samples are handled by a group of G = 2^g_log2 >= L*P consecutive lanes
// (G <= 64): lane j of the group owns sample j. The group's max, sum and dot products are
// xor-butterfly reductions, so every lane of a group holds the same bits. With L*P > 64
// (g_log2 < 0) one thread owns a unit and loops over its samples.
template <typename F>
__device__ inline float group_reduce(float x, int g, F op) {
  for (int o = g >> 1; o > 0; o >>= 1) x = op(x, __shfl_xor(x, o));
  return x;
}

struct MaxOp {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct SumOp {
  __device__ float operator()(float a, float b) const { return a + b; }
};

// 1 / extent of level l along axis d (x: W, y: H, z: D), fp32 and correctly rounded: from
// the device shapes when the host has none, with the fused forward's division.
template <int DIM>
__device__ inline float inv_at(const FusedArgs& a, uint32_t l, int d) {
  if (a.shapes) return 1.0f / (float)a.shapes[l * DIM + (DIM - 1 - d)];
  return a.inv[l][d];
}

// loc of sample i (unit u, sample j of the unit, level l) from its offsets and the
// reference point of (b, q, l)
template <int DIM, typename EI>
__device__ inline void form_loc(const FusedArgs& a, uint32_t i, uint32_t u, uint32_t l) {
  const uint32_t bq = u / (uint32_t)a.H;
  const float* r = a.ref + (bq * (uint32_t)a.L + l) * DIM;
#pragma unroll
  for (int d = 0; d < DIM; ++d)
    a.loc[i * DIM + d] = __builtin_fmaf(ld<EI>(a.off, i * DIM + d), inv_at<DIM>(a, l, d), r[d]);
}

template <int DIM, typename EI>
__global__ __launch_bounds__(kBlock) void fused_prep_kernel(const FusedArgs a) {
  const uint32_t LP = (uint32_t)(a.L * a.P);
  const uint32_t t = blockIdx.x * kBlock + threadIdx.x;
  if (a.g_log2 >= 0) {
    const int g = 1 << a.g_log2;
    const uint32_t u = t >> a.g_log2, j = t & (uint32_t)(g - 1);
    if (u >= a.units) return;  // whole groups: the grid is a multiple of G lanes
    const bool live = j < LP;
    const uint32_t i = u * LP + j;
    const float x = live ? ld<EI>(a.logits, i) : -INFINITY;
    const float m = group_reduce(x, g, MaxOp());
    const float e = live ? expf(x - m) : 0.0f;
    const float inv_sum = 1.0f / group_reduce(e, g, SumOp());
    if (!live) return;
    a.attn[i] = e * inv_sum;
    form_loc<DIM, EI>(a, i, u, j / (uint32_t)a.P);
    return;
  }
  if (t >= a.units) return;
  const uint32_t o = t * LP;
  float m = -INFINITY;
  for (uint32_t s = 0; s < LP; ++s) m = fmaxf(m, ld<EI>(a.logits, o + s));
  float sum = 0.0f;
  for (uint32_t s = 0; s < LP; ++s) sum += expf(ld<EI>(a.logits, o + s) - m);
  const float inv_sum = 1.0f / sum;
  for (uint32_t s = 0; s < LP; ++s) {
    a.attn[o + s] = expf(ld<EI>(a.logits, o + s) - m) * inv_sum;
    form_loc<DIM, EI>(a, o + s, t, s / (uint32_t)a.P);
  }
}

// Threads [0, nunit): logit and offset gradients (lane groups as above, or one thread per
// unit). Threads beyond: one (b, q, l, d) reference-point gradient each, summed over h,
// then over p.
template <int DIM, typename EI>
__global__ __launch_bounds__(kBlock) void fused_grad_kernel(const FusedArgs a) {
  const uint32_t LP = (uint32_t)(a.L * a.P);
  const uint32_t t = blockIdx.x * kBlock + threadIdx.x;
  const uint32_t nunit = a.g_log2 >= 0 ? (a.units << a.g_log2) : a.units;
  if (t < nunit) {
    if (a.g_log2 >= 0) {
      const int g = 1 << a.g_log2;
      const uint32_t u = t >> a.g_log2, j = t & (uint32_t)(g - 1);
      const bool live = j < LP;
      const uint32_t i = u * LP + j;
      const float at = live ? a.attn[i] : 0.0f, ga = live ? a.grad_attn[i] : 0.0f;
      const float dot = group_reduce(at * ga, g, SumOp());
      if (!live) return;
      st<EI>(a.grad_logits, i, at * (ga - dot));
      const uint32_t l = j / (uint32_t)a.P;
#pragma unroll
      for (int d = 0; d < DIM; ++d) st<EI>(a.grad_off, i * DIM + d, a.grad_loc[i * DIM + d] * inv_at<DIM>(a, l, d));
      return;
    }
    const uint32_t o = t * LP;
    float dot = 0.0f;
    for (uint32_t s = 0; s < LP; ++s) dot += a.attn[o + s] * a.grad_attn[o + s];
    for (uint32_t s = 0; s < LP; ++s) {
      st<EI>(a.grad_logits, o + s, a.attn[o + s] * (a.grad_attn[o + s] - dot));
      const uint32_t l = s / (uint32_t)a.P;
#pragma unroll
      for (int d = 0; d < DIM; ++d)
        st<EI>(a.grad_off, (o + s) * DIM + d, a.grad_loc[(o + s) * DIM + d] * inv_at<DIM>(a, l, d));
    }
    return;
  }
  const uint32_t jr = t - nunit;  // (b, q, l, d)
  if (jr >= a.bq * (uint32_t)a.L * DIM) return;
  const uint32_t bql = jr / DIM, d = jr - bql * DIM;
  const uint32_t bq = bql / (uint32_t)a.L, l = bql - bq * (uint32_t)a.L;
  float g = 0.0f;
  for (int h = 0; h < a.H; ++h) {
    const float* src = a.grad_loc + ((bq * (uint32_t)a.H + h) * LP + l * (uint32_t)a.P) * DIM + d;
    // the point loop's loads are independent: issue four before adding them in order
    int p = 0;
    for (; p + 4 <= a.P; p += 4) {
      const float v0 = src[p * DIM], v1 = src[(p + 1) * DIM], v2 = src[(p + 2) * DIM], v3 = src[(p + 3) * DIM];
      g += v0;
      g += v1;
      g += v2;
      g += v3;
    }
    for (; p < a.P; ++p) g += src[p * DIM];
  }
  a.grad_ref[jr] = g;
}

template <int DIM, typename EI>
hipError_t launch_both(const FusedArgs& a, bool grad, hipStream_t s) {
  const uint64_t nunit = a.g_log2 >= 0 ? ((uint64_t)a.units << a.g_log2) : a.units;
  const uint64_t n = nunit + (grad ? (uint64_t)a.bq * a.L * DIM : 0);
  if (n == 0) return hipSuccess;
  const uint32_t blocks = (uint32_t)((n + kBlock - 1) / kBlock);
  if (grad) hipLaunchKernelGGL((fused_grad_kernel<DIM, EI>), dim3(blocks), dim3(kBlock), 0, s, a);
  else hipLaunchKernelGGL((fused_prep_kernel<DIM, EI>), dim3(blocks), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fused(const FusedArgs& a, int dim, int cdt, bool grad, hipStream_t s) {
  if (dim == 2) {
    if (cdt == 0) return launch_both<2, F32>(a, grad, s);
    if (cdt == 1) return launch_both<2, F16>(a, grad, s);
    if (cdt == 2) return launch_both<2, BF16>(a, grad, s);
  } else if (dim == 3) {
    if (cdt == 0) return launch_both<3, F32>(a, grad, s);
    if (cdt == 1) return launch_both<3, F16>(a, grad, s);
    if (cdt == 2) return launch_both<3, BF16>(a, grad, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace msda
