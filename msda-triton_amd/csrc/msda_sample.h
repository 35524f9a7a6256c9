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

// Tile (along one axis, extent T = 2^t_log2 cells) that owns a sample's lowest valid
// corner; the sample must have a valid corner on this axis (i0 >= -1). Its corners i0 and
// i0 + 1 then lie in [tile * T - 1, tile * T + T]: the tile or its one-cell high-side halo.
__device__ inline int anchor_tile(const Axis& a, int t_log2) { return (a.i0 < 0 ? 0 : a.i0) >> t_log2; }

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

// ---------------------------------------------------------------------------------------
// Coordinate / weight blocks: the N consecutive coordinate-type elements of a batch of
// samples, read with the widest loads their alignment allows (callers guarantee the
// block start is aligned to the block size, up to 16 bytes).
template <typename EC, int N>
struct CoordBlock {
  static constexpr int kBytes = N * EC::kBytes;
  static constexpr int kDwords = (kBytes + 3) / 4;
  uint32_t d[kDwords];
};

template <typename EC, int N>
__device__ inline void load_block(CoordBlock<EC, N>& b, const typename EC::T* p) {
  constexpr int B = CoordBlock<EC, N>::kBytes;
  if constexpr (B % 16 == 0) {
#pragma unroll
    for (int i = 0; i < B / 16; ++i) {
      const u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
      b.d[4 * i] = v[0];
      b.d[4 * i + 1] = v[1];
      b.d[4 * i + 2] = v[2];
      b.d[4 * i + 3] = v[3];
    }
  } else if constexpr (B % 8 == 0) {
#pragma unroll
    for (int i = 0; i < B / 8; ++i) {
      const u32x2 v = reinterpret_cast<const u32x2*>(p)[i];
      b.d[2 * i] = v[0];
      b.d[2 * i + 1] = v[1];
    }
  } else if constexpr (B % 4 == 0) {
#pragma unroll
    for (int i = 0; i < B / 4; ++i) b.d[i] = reinterpret_cast<const uint32_t*>(p)[i];
  } else {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i & 1) b.d[i / 2] |= (uint32_t)h[i] << 16;
      else b.d[i / 2] = h[i];
    }
  }
}

// Store N fp32 values as a block of EC elements (round to nearest even), with the widest
// stores the alignment allows.
template <typename EC, int N>
__device__ inline void store_block(typename EC::T* p, const float (&v)[N]) {
  constexpr int B = N * EC::kBytes;
  uint32_t d[(B + 3) / 4];
  if constexpr (EC::kBytes == 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) d[i] = __builtin_bit_cast(uint32_t, v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < (N + 1) / 2; ++i) {
      const uint32_t lo = __builtin_bit_cast(uint16_t, narrow<EC>(v[2 * i]));
      const uint32_t hi = 2 * i + 1 < N ? __builtin_bit_cast(uint16_t, narrow<EC>(v[2 * i + 1])) : 0u;
      d[i] = lo | (hi << 16);
    }
  }
  if constexpr (B % 16 == 0) {
#pragma unroll
    for (int i = 0; i < B / 16; ++i)
      reinterpret_cast<u32x4*>(p)[i] = u32x4{d[4 * i], d[4 * i + 1], d[4 * i + 2], d[4 * i + 3]};
  } else if constexpr (B % 8 == 0) {
#pragma unroll
    for (int i = 0; i < B / 8; ++i) reinterpret_cast<u32x2*>(p)[i] = u32x2{d[2 * i], d[2 * i + 1]};
  } else if constexpr (B % 4 == 0) {
#pragma unroll
    for (int i = 0; i < B / 4; ++i) reinterpret_cast<uint32_t*>(p)[i] = d[i];
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = narrow<EC>(v[i]);
  }
}

// Element i of a block as fp32.
template <typename EC, int N>
__device__ inline float block_elem(const CoordBlock<EC, N>& b, int i) {
  if constexpr (EC::kBytes == 4) {
    return __builtin_bit_cast(float, b.d[i]);
  } else {
    const uint32_t u = b.d[i / 2];
    if constexpr (__is_same(EC, BF16)) return (i & 1) ? bf16hi(u) : bf16lo(u);
    else return (i & 1) ? f16hi(u) : f16lo(u);
  }
}

}  // namespace msda
