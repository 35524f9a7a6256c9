// msda_sample.h — per-sample sampling geometry shared by every MSDA kernel.
//
// Sampling follows torch.nn.functional.grid_sample(mode="bilinear",
// padding_mode="zeros", align_corners=False) applied to grid = 2*loc - 1, as in the
// reference's oracle msda2d_pytorch (src/msda_triton/pytorch/msda_2d.py:65-98) and
// msda3d_pytorch (src/msda_triton/pytorch/msda_3d.py:65-102). The grid is optionally
// clamped to [-1+eps, 1-eps] and mapped to the pixel coordinate u = ((g+1)*size-1)/2
// (ATen GridSampler.h grid_sampler_unnormalize, align_corners=False). The arithmetic is
// kept uncontracted so it rounds exactly like ATen's scalar formula, and so every kernel
// that recomputes a sample (forward, backward binning, backward tiles) selects the same
// corners bit for bit.
#pragma once

#include "msda_device.h"

namespace msda {

// One axis of a sample: lower corner, the two linear weights, and in-range flags.
struct Axis {
  float e;      // weight of the lower corner: (i0 + 1) - u
  float f;      // weight of the upper corner: u - i0
  int i0;       // lower corner index (floor(u) clamped to [-2, size + 1] before conversion)
  bool v0, v1;  // lower / upper corner inside [0, size)
  bool pass;    // gradient passes the grid clamp (backward mask of torch.clamp)
};

// Tile (along one axis, extent T cells) that owns a sample's lowest valid corner; the
// sample must have a valid corner on this axis (i0 >= -1). Its corners i0 and i0 + 1
// then lie in [tile * T - 1, tile * T + T]: the tile or its one-cell high-side halo.
__device__ inline int anchor_tile(const Axis& a, int T) { return (a.i0 < 0 ? 0 : a.i0) / T; }

// Pixel coordinate u of one location component; *pass is false where the grid clamp
// was active.
__device__ inline float grid_to_u(float loc, float size_f, int clamp, float lo, float hi,
                                  bool* pass) {
#pragma clang fp contract(off)
  float g = 2.0f * loc - 1.0f;
  *pass = !clamp || (g >= lo && g <= hi);
  if (clamp) g = fminf(fmaxf(g, lo), hi);
  return ((g + 1.0f) * size_f - 1.0f) * 0.5f;
}

// Corner indices, weights and validity from a pixel coordinate. Every kernel derives an
// axis through this function, so a coordinate stored by one kernel and expanded by
// another selects the same corners with the same weights.
__device__ inline Axis axis_from_u(float u, int size_i, bool pass) {
#pragma clang fp contract(off)
  Axis a;
  const float u0 = floorf(u);
  a.f = u - u0;
  a.e = (u0 + 1.0f) - u;
  a.i0 = (int)fminf(fmaxf(u0, -2.0f), (float)size_i + 1.0f);
  a.v0 = (unsigned)a.i0 < (unsigned)size_i;
  a.v1 = (unsigned)(a.i0 + 1) < (unsigned)size_i;
  a.pass = pass;
  return a;
}

__device__ inline Axis make_axis(float loc, float size_f, int size_i, int clamp, float lo,
                                 float hi) {
  bool pass;
  const float u = grid_to_u(loc, size_f, clamp, lo, hi, &pass);
  return axis_from_u(u, size_i, pass);
}

// Level table entry: first row of the level in K, and its extents (D = 1 in 2D).
struct Level {
  int32_t start, W, H, D;
};

// Corner c of a sample: bit 0 selects x0/x0+1, bit 1 y, bit 2 z.
template <int DIM>
struct Sample {
  Axis ax, ay, az;
};

template <int DIM>
__device__ inline bool corner_valid(int c, const Sample<DIM>& s) {
  bool v = (c & 1) ? s.ax.v1 : s.ax.v0;
  v = v && ((c & 2) ? s.ay.v1 : s.ay.v0);
  if constexpr (DIM == 3) v = v && ((c & 4) ? s.az.v1 : s.az.v0);
  return v;
}

template <int DIM>
__device__ inline float corner_weight(int c, const Sample<DIM>& s) {
  const float wx = (c & 1) ? s.ax.f : s.ax.e;
  const float wy = (c & 2) ? s.ay.f : s.ay.e;
  if constexpr (DIM == 3) {
    const float wz = (c & 4) ? s.az.f : s.az.e;
    return wx * wy * wz;
  } else {
    return wx * wy;
  }
}

// Build the sample's axes from its DIM coordinates (order x, y[, z]).
template <int DIM, typename TC>
__device__ inline Sample<DIM> make_sample(const TC* lp, const Level& lv, int clamp, float lo,
                                          float hi) {
  Sample<DIM> s;
  s.ax = make_axis((float)lp[0], (float)lv.W, lv.W, clamp, lo, hi);
  s.ay = make_axis((float)lp[1], (float)lv.H, lv.H, clamp, lo, hi);
  if constexpr (DIM == 3) s.az = make_axis((float)lp[2], (float)lv.D, lv.D, clamp, lo, hi);
  return s;
}

// Accumulate the per-corner dot products <grad_out, value_corner> into
// d(out)/d(attn) = sum_c w_c dot_c and d(out)/d(u_axis) = sum_c (dw_c/du) dot_c.
template <int DIM>
__device__ inline void corner_grads(const Sample<DIM>& sm, const float* dot, float& s_attn,
                                    float& s_x, float& s_y, float& s_z) {
  s_attn = s_x = s_y = s_z = 0.0f;
#pragma unroll
  for (int c = 0; c < (1 << DIM); ++c) {
    const float wx = (c & 1) ? sm.ax.f : sm.ax.e;
    const float wy = (c & 2) ? sm.ay.f : sm.ay.e;
    const float sx = (c & 1) ? 1.0f : -1.0f;
    const float sy = (c & 2) ? 1.0f : -1.0f;
    if constexpr (DIM == 3) {
      const float wz = (c & 4) ? sm.az.f : sm.az.e;
      const float sz = (c & 4) ? 1.0f : -1.0f;
      s_attn += wx * wy * wz * dot[c];
      s_x += sx * wy * wz * dot[c];
      s_y += wx * sy * wz * dot[c];
      s_z += wx * wy * sz * dot[c];
    } else {
      s_attn += wx * wy * dot[c];
      s_x += sx * wy * dot[c];
      s_y += wx * sy * dot[c];
    }
  }
}

}  // namespace msda
