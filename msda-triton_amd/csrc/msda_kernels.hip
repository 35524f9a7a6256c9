// msda_kernels.hip — gfx950 forward and backward kernels for multi-scale deformable
// attention with bilinear (2D) and trilinear (3D) sampling.
//
// Work decomposition (both kernels). A "unit" is one (batch b, query q, head h).
// Each unit is owned by an aligned group of 2^lpu_log2 lanes of one wave64. Lane j
// of the group holds channels [j*VEC, (j+1)*VEC) of the unit, so every corner of a
// sample is fetched as one VEC*sizeof(value) byte load per lane (16 B when C allows).
// The lanes of a unit together read one contiguous C-channel value row. Units are
// enumerated in (b, head-group, q, head-in-group) order: the 2^hg_log2 heads of a
// group share the 128-byte lines of value, loc, attn and output rows. Workgroups are
// remapped so that each XCD owns a contiguous unit range, which keeps a
// (batch, head-group) value slice resident in that XCD's L2.
//
// Sampling follows torch.nn.functional.grid_sample(mode="bilinear",
// padding_mode="zeros", align_corners=False) applied to grid = 2*loc - 1, as in the
// reference's oracle msda2d_pytorch (src/msda_triton/pytorch/msda_2d.py:65-98) and
// msda3d_pytorch (src/msda_triton/pytorch/msda_3d.py:65-102). The grid is optionally
// clamped to [-1+eps, 1-eps], and its pixel coordinate is ((g+1)*size-1)/2
// (ATen GridSampler.h grid_sampler_unnormalize). The coordinate arithmetic is kept
// uncontracted so that it rounds exactly like ATen's scalar formula. Corners outside
// the level read as zero through the buffer range check.
#include "msda_internal.h"

namespace msda {

namespace {

// One axis of a sample: floor corner, the two linear weights, and in-range flags.
struct Axis {
  float e;     // weight of the lower corner: (i0 + 1) - u
  float f;     // weight of the upper corner: u - i0
  int i0;      // lower corner index (clamped to [-2, size + 1] before conversion)
  bool v0, v1; // lower / upper corner inside [0, size)
  bool pass;   // gradient passes the grid clamp (torch.clamp backward mask)
};

__device__ inline Axis make_axis(float loc, float size_f, int size_i, int clamp, float lo,
                                 float hi) {
#pragma clang fp contract(off)
  Axis a;
  float g = 2.0f * loc - 1.0f;
  a.pass = !clamp || (g >= lo && g <= hi);
  if (clamp) g = fminf(fmaxf(g, lo), hi);
  const float u = ((g + 1.0f) * size_f - 1.0f) * 0.5f;
  const float u0 = floorf(u);
  a.f = u - u0;
  a.e = (u0 + 1.0f) - u;
  a.i0 = (int)fminf(fmaxf(u0, -2.0f), size_f + 1.0f);
  a.v0 = (unsigned)a.i0 < (unsigned)size_i;
  a.v1 = (unsigned)(a.i0 + 1) < (unsigned)size_i;
  return a;
}

struct Unit {
  uint32_t b, q, h, lane, bqh;
};

__device__ inline bool decode_unit(const Params& p, Unit& u) {
  const uint32_t lb = xcd_logical_block(blockIdx.x, p.nblocks);
  const uint32_t t = lb * kBlock + threadIdx.x;
  const uint32_t unit = t >> p.lpu_log2;
  u.lane = t & ((1u << p.lpu_log2) - 1u);
  if (unit >= p.num_units) return false;
  u.b = fdiv(unit, p.div_qh);
  const uint32_t r = unit - u.b * p.div_qh.d;
  const uint32_t hgrp = fdiv(r, p.div_qhg);
  const uint32_t r2 = r - hgrp * p.div_qhg.d;
  u.q = r2 >> p.hg_log2;
  u.h = (hgrp << p.hg_log2) | (r2 & ((1u << p.hg_log2) - 1u));
  u.bqh = (u.b * p.Q + u.q) * (uint32_t)p.H + u.h;
  return true;
}

// Level table: x = first row of the level in K, y = W, z = H, w = D (1 for 2D).
template <int DIM>
__device__ inline void stage_levels(const Params& p, int4* s_lvl) {
  for (int i = threadIdx.x; i < p.L; i += kBlock) {
    int4 e;
    e.x = p.starts[i];
    if constexpr (DIM == 2) {
      e.w = 1;
      e.z = p.shapes[2 * i];
      e.y = p.shapes[2 * i + 1];
    } else {
      e.w = p.shapes[3 * i];
      e.z = p.shapes[3 * i + 1];
      e.y = p.shapes[3 * i + 2];
    }
    s_lvl[i] = e;
  }
}

// Per-sample geometry shared by forward and backward.
template <int DIM>
struct Sample {
  static constexpr int NC = 1 << DIM;
  Axis ax, ay, az;
  uint32_t row0;  // row index (in K) of the all-lower corner, modulo 2^32
};

template <int DIM>
__device__ inline uint32_t corner_row_delta(int c, uint32_t W, uint32_t HW) {
  return ((c & 1) ? 1u : 0u) + ((c & 2) ? W : 0u) + ((DIM == 3 && (c & 4)) ? HW : 0u);
}

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

}  // namespace

// ---------------------------------------------------------------------------------------
// Forward. Replaces the reference's _fwd_kernel_2d (src/msda_triton/triton/msda_2d.py:85-260)
// and _fwd_kernel (src/msda_triton/triton/msda_3d.py:80-288), and writes (B, Q, H*C) in the
// value dtype directly instead of an fp32 (B*H, Q, C) scratch plus permute (msda_2d.py:649-651).
template <int DIM, typename EV, typename EC, int VEC>
__global__ __launch_bounds__(kBlock) void msda_fwd_kernel(const Params p) {
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  typedef typename EC::T TC;
  __shared__ int4 s_lvl[kMaxLevels];
  stage_levels<DIM>(p, s_lvl);
  __syncthreads();

  Unit u;
  if (!decode_unit(p, u)) return;
  if ((int)u.lane >= p.nvec) return;

  const int LP = p.L * p.P;
  const TC* locp = static_cast<const TC*>(p.loc) + (size_t)u.bqh * (LP * DIM);
  const TC* attp = static_cast<const TC*>(p.attn) + (size_t)u.bqh * LP;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.value, p.value_bytes);
  const uint32_t rs = (uint32_t)p.H * (uint32_t)p.C * EV::kBytes;  // bytes between rows of K
  const uint32_t vbase =
      ((u.b * (uint32_t)p.K * (uint32_t)p.H + u.h) * (uint32_t)p.C + u.lane * VEC) * EV::kBytes;

  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;

  for (int l = 0; l < p.L; ++l) {
    const int4 e = s_lvl[l];
    const uint32_t W = (uint32_t)e.y, HW = (uint32_t)e.y * (uint32_t)e.z;
    const float fW = (float)e.y, fH = (float)e.z, fD = (float)e.w;
    for (int pp = 0; pp < p.P; ++pp) {
      const int s = l * p.P + pp;
      const float a = (float)attp[s];
      Sample<DIM> sm;
      sm.ax = make_axis((float)locp[s * DIM + 0], fW, e.y, p.clamp, p.lo_g, p.hi_g);
      sm.ay = make_axis((float)locp[s * DIM + 1], fH, e.z, p.clamp, p.lo_g, p.hi_g);
      uint32_t row0 = (uint32_t)e.x + (uint32_t)sm.ay.i0 * W + (uint32_t)sm.ax.i0;
      if constexpr (DIM == 3) {
        sm.az = make_axis((float)locp[s * DIM + 2], fD, e.w, p.clamp, p.lo_g, p.hi_g);
        row0 += (uint32_t)sm.az.i0 * HW;
      }
      const uint32_t off0 = vbase + row0 * rs;

      RawVec<VB> raw[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint32_t off = off0 + corner_row_delta<DIM>(c, W, HW) * rs;
        raw[c] = buf_load<VB>(rv, corner_valid<DIM>(c, sm) ? off : kOobOffset);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float cw = corner_weight<DIM>(c, sm) * a;
        float v[VEC];
        widen<EV, VEC>(raw[c], v);
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[i] = __builtin_fmaf(cw, v[i], acc[i]);
      }
    }
  }
  typename EV::T* outp = static_cast<typename EV::T*>(p.out) + (size_t)u.bqh * p.C + u.lane * VEC;
  store_vec<EV, VEC>(outp, acc);
}

// ---------------------------------------------------------------------------------------
// Backward. Replaces _bwd_kernel_2d (src/msda_triton/triton/msda_2d.py:263-510) and the 3D
// _bwd_kernel (src/msda_triton/triton/msda_3d.py:291-653). One lane group owns a unit, so
// grad_sampling_locations and grad_attention_weights are reduced across the group with
// lane exchanges and written with plain stores; grad_value is scattered with fp32 buffer
// atomics (no-return), whose out-of-range offset drops the add for corners outside the
// level. grad_output is read once per unit rather than once per (level, point).
template <int DIM, typename EV, typename EC, int VEC>
__global__ __launch_bounds__(kBlock) void msda_bwd_kernel(const Params p) {
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  typedef typename EC::T TC;
  __shared__ int4 s_lvl[kMaxLevels];
  stage_levels<DIM>(p, s_lvl);
  __syncthreads();

  Unit u;
  if (!decode_unit(p, u)) return;
  // Lanes past C/VEC stay in the loop (they take part in the group reductions) but
  // load zeros and never write.
  const bool act = (int)u.lane < p.nvec;
  const int lg = p.lpu_log2;

  float g[VEC];
  {
    const typename EV::T* gop =
        static_cast<const typename EV::T*>(p.grad_out) + (size_t)u.bqh * p.C + u.lane * VEC;
    if (act) {
      RawVec<VB> r = glb_load<VB>(gop);
      widen<EV, VEC>(r, g);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) g[i] = 0.0f;
    }
  }

  const int LP = p.L * p.P;
  const TC* locp = static_cast<const TC*>(p.loc) + (size_t)u.bqh * (LP * DIM);
  const TC* attp = static_cast<const TC*>(p.attn) + (size_t)u.bqh * LP;
  TC* gl = static_cast<TC*>(p.grad_loc) + (size_t)u.bqh * (LP * DIM);
  TC* ga = static_cast<TC*>(p.grad_attn) + (size_t)u.bqh * LP;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.value, p.value_bytes);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.grad_acc, p.acc_bytes);
  const uint32_t rs = (uint32_t)p.H * (uint32_t)p.C * EV::kBytes;
  const uint32_t rsa = (uint32_t)p.H * (uint32_t)p.C * 4u;
  const uint32_t ebase = (u.b * (uint32_t)p.K * (uint32_t)p.H + u.h) * (uint32_t)p.C + u.lane * VEC;
  const uint32_t vbase = ebase * EV::kBytes;
  const uint32_t abase = ebase * 4u;

  for (int l = 0; l < p.L; ++l) {
    const int4 e = s_lvl[l];
    const uint32_t W = (uint32_t)e.y, HW = (uint32_t)e.y * (uint32_t)e.z;
    const float fW = (float)e.y, fH = (float)e.z, fD = (float)e.w;
    for (int pp = 0; pp < p.P; ++pp) {
      const int s = l * p.P + pp;
      const float a = (float)attp[s];
      Sample<DIM> sm;
      sm.ax = make_axis((float)locp[s * DIM + 0], fW, e.y, p.clamp, p.lo_g, p.hi_g);
      sm.ay = make_axis((float)locp[s * DIM + 1], fH, e.z, p.clamp, p.lo_g, p.hi_g);
      uint32_t row0 = (uint32_t)e.x + (uint32_t)sm.ay.i0 * W + (uint32_t)sm.ax.i0;
      if constexpr (DIM == 3) {
        sm.az = make_axis((float)locp[s * DIM + 2], fD, e.w, p.clamp, p.lo_g, p.hi_g);
        row0 += (uint32_t)sm.az.i0 * HW;
      }

      RawVec<VB> raw[NC];
      uint32_t aoff[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint32_t dr = row0 + corner_row_delta<DIM>(c, W, HW);
        const bool ok = act && corner_valid<DIM>(c, sm);
        raw[c] = buf_load<VB>(rv, ok ? vbase + dr * rs : kOobOffset);
        aoff[c] = ok ? abase + dr * rsa : kOobOffset;
      }

      // grad_value scatter: attn * w_corner * grad_out
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float cw = corner_weight<DIM>(c, sm) * a;
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(cw * g[i], ra, (int)(aoff[c] + 4u * i),
                                                          0, 0);
      }

      // dot[c] = <grad_out, value row of corner c> over this lane's channels
      float dot[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float v[VEC];
        widen<EV, VEC>(raw[c], v);
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) d = __builtin_fmaf(g[i], v[i], d);
        dot[c] = d;
      }

      // d(out)/d(attn) = sum_c w_c dot_c ; d(out)/d(u_axis) = sum_c (dw_c/du) dot_c
      float s_attn = 0.0f, s_x = 0.0f, s_y = 0.0f, s_z = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
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
      s_attn = group_sum(s_attn, lg);
      s_x = group_sum(s_x, lg);
      s_y = group_sum(s_y, lg);
      if constexpr (DIM == 3) s_z = group_sum(s_z, lg);

      if (u.lane == 0) {
        ga[s] = (TC)s_attn;
        gl[s * DIM + 0] = (TC)(sm.ax.pass ? (a * s_x) * fW : 0.0f);
        gl[s * DIM + 1] = (TC)(sm.ay.pass ? (a * s_y) * fH : 0.0f);
        if constexpr (DIM == 3) gl[s * DIM + 2] = (TC)(sm.az.pass ? (a * s_z) * fD : 0.0f);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Clears n floats. vec selects 16-byte stores (p must then be 16-byte aligned).
__global__ __launch_bounds__(kBlock) void fill_zero_kernel(float* p, size_t n, int vec) {
  const size_t n4 = vec ? n / 4 : 0;
  float4* p4 = reinterpret_cast<float4*>(p);
  const size_t stride = (size_t)gridDim.x * kBlock;
  const size_t t0 = (size_t)blockIdx.x * kBlock + threadIdx.x;
  for (size_t i = t0; i < n4; i += stride) p4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (size_t i = n4 * 4 + t0; i < n; i += stride) p[i] = 0.0f;
}

// dst[i] = (value dtype) src[i], round to nearest even. vec: dst is 8-byte aligned.
template <typename EV>
__global__ __launch_bounds__(kBlock) void narrow_kernel(const float* src, typename EV::T* dst,
                                                         size_t n, int vec) {
  const size_t n4 = vec ? n / 4 : 0;
  const size_t stride = (size_t)gridDim.x * kBlock;
  const size_t t0 = (size_t)blockIdx.x * kBlock + threadIdx.x;
  typedef typename EV::T T;
  typedef T t4 __attribute__((ext_vector_type(4)));
  for (size_t i = t0; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4*>(src)[i];
    t4 o;
    o[0] = (T)v.x;
    o[1] = (T)v.y;
    o[2] = (T)v.z;
    o[3] = (T)v.w;
    reinterpret_cast<t4*>(dst)[i] = o;
  }
  for (size_t i = n4 * 4 + t0; i < n; i += stride) dst[i] = (T)src[i];
}

static unsigned elementwise_blocks(size_t n) {
  size_t b = (n / 4 + kBlock - 1) / kBlock;
  if (b < 1) b = 1;
  if (b > 8192) b = 8192;
  return (unsigned)b;
}

hipError_t launch_fill_zero(float* p, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const int vec = ((uintptr_t)p % 16) == 0;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(elementwise_blocks(n)), dim3(kBlock), 0, s, p, n, vec);
  return hipGetLastError();
}

hipError_t launch_narrow(const float* src, void* dst, int vdt, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const dim3 grid(elementwise_blocks(n));
  const int vec = ((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 8) == 0;
  if (vdt == 1)
    hipLaunchKernelGGL(narrow_kernel<F16>, grid, dim3(kBlock), 0, s, src,
                       static_cast<_Float16*>(dst), n, vec);
  else
    hipLaunchKernelGGL(narrow_kernel<BF16>, grid, dim3(kBlock), 0, s, src,
                       static_cast<__bf16*>(dst), n, vec);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Launcher tables.
template <int DIM, typename EV, typename EC, int VEC>
static hipError_t launch_fwd(const Params& p, hipStream_t s) {
  hipLaunchKernelGGL((msda_fwd_kernel<DIM, EV, EC, VEC>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  return hipGetLastError();
}

template <int DIM, typename EV, typename EC, int VEC>
static hipError_t launch_bwd(const Params& p, hipStream_t s) {
  hipLaunchKernelGGL((msda_bwd_kernel<DIM, EV, EC, VEC>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  return hipGetLastError();
}

template <bool FWD, int DIM, typename EV, typename EC>
static LaunchFn pick_vec(int vec_bytes) {
  constexpr int S = EV::kBytes;
  switch (vec_bytes) {
    case 16:
      return FWD ? &launch_fwd<DIM, EV, EC, 16 / S> : &launch_bwd<DIM, EV, EC, 16 / S>;
    case 8:
      return FWD ? &launch_fwd<DIM, EV, EC, 8 / S> : &launch_bwd<DIM, EV, EC, 8 / S>;
    case 4:
      return FWD ? &launch_fwd<DIM, EV, EC, 4 / S> : &launch_bwd<DIM, EV, EC, 4 / S>;
    case 2:
      if constexpr (S == 2) return FWD ? &launch_fwd<DIM, EV, EC, 1> : &launch_bwd<DIM, EV, EC, 1>;
      return nullptr;
    default:
      return nullptr;
  }
}

template <bool FWD, int DIM>
static LaunchFn pick_types(int vdt, int cdt, int vec_bytes) {
  if (vdt == 0 && cdt == 0) return pick_vec<FWD, DIM, F32, F32>(vec_bytes);
  if (vdt == 1 && cdt == 1) return pick_vec<FWD, DIM, F16, F16>(vec_bytes);
  if (vdt == 1 && cdt == 0) return pick_vec<FWD, DIM, F16, F32>(vec_bytes);
  if (vdt == 2 && cdt == 2) return pick_vec<FWD, DIM, BF16, BF16>(vec_bytes);
  if (vdt == 2 && cdt == 0) return pick_vec<FWD, DIM, BF16, F32>(vec_bytes);
  return nullptr;
}

LaunchFn get_fwd_launcher(int dim, int vdt, int cdt, int vec_bytes) {
  if (dim == 2) return pick_types<true, 2>(vdt, cdt, vec_bytes);
  if (dim == 3) return pick_types<true, 3>(vdt, cdt, vec_bytes);
  return nullptr;
}

LaunchFn get_bwd_launcher(int dim, int vdt, int cdt, int vec_bytes) {
  if (dim == 2) return pick_types<false, 2>(vdt, cdt, vec_bytes);
  if (dim == 3) return pick_types<false, 3>(vdt, cdt, vec_bytes);
  return nullptr;
}

}  // namespace msda
