// msda_fwd.hip — gfx950 forward kernel: bilinear (2D) / trilinear (3D) multi-scale
// deformable attention.
//
// Work decomposition. A "unit" is one (batch b, query q, head h), owned by an aligned
// group of 2^lpu_log2 lanes of one wave64. Lane j of the group holds channels
// [j*VEC, (j+1)*VEC), so each corner of a sample is one VEC*sizeof(value)-byte load per
// lane (16 B when C allows) and the group together reads one contiguous C-channel value
// row. Units are enumerated in (b, head-group, q, head-in-group) order so the heads that
// share 128-byte lines of value/loc/attn/output rows run side by side, and workgroups are
// remapped so each XCD owns a contiguous unit range, keeping a (batch, head-group) value
// slice resident in that XCD's L2. Samples are processed in batches of SB: all SB*2^DIM
// corner loads of a batch are issued before any is consumed, which keeps 16 row loads in
// flight per lane. Corners outside the level read as zero through the buffer range check;
// accumulation is fp32 and the output is rounded once to the value dtype.
#include "msda_internal.h"
#include "msda_sample.h"

namespace msda {

namespace {

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

template <int DIM>
__device__ inline void stage_levels(const Params& p, Level* s_lvl) {
  for (int i = threadIdx.x; i < p.L; i += kBlock) {
    Level e;
    e.start = p.starts[i];
    if constexpr (DIM == 2) {
      e.D = 1;
      e.H = p.shapes[2 * i];
      e.W = p.shapes[2 * i + 1];
    } else {
      e.D = p.shapes[3 * i];
      e.H = p.shapes[3 * i + 1];
      e.W = p.shapes[3 * i + 2];
    }
    s_lvl[i] = e;
  }
}

}  // namespace

// Replaces the reference's _fwd_kernel_2d (src/msda_triton/triton/msda_2d.py:85-260) and
// _fwd_kernel (src/msda_triton/triton/msda_3d.py:80-288). Writes (B, Q, H*C) in the value
// dtype directly instead of an fp32 (B*H, Q, C) scratch plus permute (msda_2d.py:649-651).
//
// PT > 0: the number of points per level is a compile-time constant. Each level's PT*DIM
// coordinates and PT weights are fetched as one contiguous block per lane, the next
// level's block is fetched while this level's corner rows are in flight, and all corner
// rows of a level (in batches of SB samples) are issued before any is consumed; the
// in-order completion of vector loads then never makes a coordinate load wait behind a
// row gather. PT == 0 handles any P with per-sample loads.
template <int DIM, typename EV, typename EC, int VEC, int PT>
__global__ __launch_bounds__(kBlock) void msda_fwd_kernel(const Params p) {
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  constexpr int SB = PT > 0 ? (DIM == 2 ? (PT < 4 ? PT : 4) : (PT < 2 ? PT : 2)) : (DIM == 2 ? 4 : 2);
  typedef typename EC::T TC;
  __shared__ Level s_lvl[kMaxLevels];
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

  if constexpr (PT > 0) {
    // Software pipeline over batches of SB samples (all levels, in order): the batch's
    // coordinates and weights were fetched during the previous iteration.
    constexpr int BPL = PT / SB;  // batches per level
    CoordBlock<EC, SB * DIM> lb;
    CoordBlock<EC, SB> ab;
    const int nbatch = p.L * BPL;
    if (nbatch > 0) {
      load_block<EC, SB * DIM>(lb, locp);
      load_block<EC, SB>(ab, attp);
    }
#pragma unroll 1
    for (int bi = 0; bi < nbatch; ++bi) {
      const Level lv = s_lvl[bi / BPL];
      const uint32_t W = (uint32_t)lv.W, HW = (uint32_t)lv.W * (uint32_t)lv.H;
      uint32_t off[SB][NC];
      float cw[SB][NC];
#pragma unroll
      for (int k = 0; k < SB; ++k) {
        Sample<DIM> sm;
        sm.ax = make_axis(block_elem(lb, k * DIM + 0), (float)lv.W, lv.W, p.clamp, p.lo_g, p.hi_g);
        sm.ay = make_axis(block_elem(lb, k * DIM + 1), (float)lv.H, lv.H, p.clamp, p.lo_g, p.hi_g);
        uint32_t row0 = (uint32_t)lv.start + (uint32_t)sm.ay.i0 * W + (uint32_t)sm.ax.i0;
        if constexpr (DIM == 3) {
          sm.az = make_axis(block_elem(lb, k * DIM + 2), (float)lv.D, lv.D, p.clamp, p.lo_g, p.hi_g);
          row0 += (uint32_t)sm.az.i0 * HW;
        }
        const float a = block_elem(ab, k);
        const uint32_t off0 = vbase + row0 * rs;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const uint32_t dr = ((c & 1) ? 1u : 0u) + ((c & 2) ? W : 0u) + ((DIM == 3 && (c & 4)) ? HW : 0u);
          off[k][c] = corner_valid<DIM>(c, sm) ? off0 + dr * rs : kOobOffset;
          cw[k][c] = corner_weight<DIM>(c, sm) * a;
        }
      }
      RawVec<VB> raw[SB][NC];
#pragma unroll
      for (int k = 0; k < SB; ++k)
#pragma unroll
        for (int c = 0; c < NC; ++c) raw[k][c] = buf_load<VB>(rv, off[k][c]);
      if (bi + 1 < nbatch) {
        // next batch's coordinates and weights, queued behind this batch's rows
        load_block<EC, SB * DIM>(lb, locp + (bi + 1) * (SB * DIM));
        load_block<EC, SB>(ab, attp + (bi + 1) * SB);
      }
#pragma unroll
      for (int k = 0; k < SB; ++k) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float v[VEC];
          widen<EV, VEC>(raw[k][c], v);
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] = __builtin_fmaf(cw[k][c], v[i], acc[i]);
        }
      }
    }
  } else {
    for (int l = 0; l < p.L; ++l) {
      const Level lv = s_lvl[l];
      const uint32_t W = (uint32_t)lv.W, HW = (uint32_t)lv.W * (uint32_t)lv.H;
      for (int p0 = 0; p0 < p.P; p0 += SB) {
        RawVec<VB> raw[SB][NC];
        float cw[SB][NC];
#pragma unroll
        for (int k = 0; k < SB; ++k) {
          const int s = l * p.P + p0 + k;
          const bool live = p0 + k < p.P;
          const float a = live ? (float)attp[s] : 0.0f;
          const Sample<DIM> sm =
              make_sample<DIM>(locp + (live ? s : 0) * DIM, lv, p.clamp, p.lo_g, p.hi_g);
          uint32_t row0 = (uint32_t)lv.start + (uint32_t)sm.ay.i0 * W + (uint32_t)sm.ax.i0;
          if constexpr (DIM == 3) row0 += (uint32_t)sm.az.i0 * HW;
          const uint32_t off0 = vbase + row0 * rs;
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const uint32_t dr = ((c & 1) ? 1u : 0u) + ((c & 2) ? W : 0u) +
                                ((DIM == 3 && (c & 4)) ? HW : 0u);
            raw[k][c] = buf_load<VB>(rv, (live && corner_valid<DIM>(c, sm)) ? off0 + dr * rs : kOobOffset);
            cw[k][c] = corner_weight<DIM>(c, sm) * a;
          }
        }
#pragma unroll
        for (int k = 0; k < SB; ++k) {
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            float v[VEC];
            widen<EV, VEC>(raw[k][c], v);
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[i] = __builtin_fmaf(cw[k][c], v[i], acc[i]);
          }
        }
        // keep the compiler from hoisting the next batch's row loads above these FMAs,
        // which would multiply the live row registers and cut occupancy
        asm volatile("" ::: "memory");
      }
    }
  }
  typename EV::T* outp = static_cast<typename EV::T*>(p.out) + (size_t)u.bqh * p.C + u.lane * VEC;
  store_vec<EV, VEC>(outp, acc);
}

template <int DIM, typename EV, typename EC, int VEC>
static hipError_t launch_fwd(const Params& p, hipStream_t s) {
  // compile-time point counts for the common 4 and 8 points per level
  if (p.P == 4 && p.coords_aligned)
    hipLaunchKernelGGL((msda_fwd_kernel<DIM, EV, EC, VEC, 4>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  else if (p.P == 8 && p.coords_aligned)
    hipLaunchKernelGGL((msda_fwd_kernel<DIM, EV, EC, VEC, 8>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  else
    hipLaunchKernelGGL((msda_fwd_kernel<DIM, EV, EC, VEC, 0>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  return hipGetLastError();
}

template <int DIM, typename EV, typename EC>
static LaunchFn pick_vec(int vec_bytes) {
  constexpr int S = EV::kBytes;
  switch (vec_bytes) {
    case 16: return &launch_fwd<DIM, EV, EC, 16 / S>;
    case 8: return &launch_fwd<DIM, EV, EC, 8 / S>;
    case 4: return &launch_fwd<DIM, EV, EC, 4 / S>;
    case 2:
      if constexpr (S == 2) return &launch_fwd<DIM, EV, EC, 1>;
      return nullptr;
    default: return nullptr;
  }
}

template <int DIM>
static LaunchFn pick_types(int vdt, int cdt, int vec_bytes) {
  if (vdt == 0 && cdt == 0) return pick_vec<DIM, F32, F32>(vec_bytes);
  if (vdt == 1 && cdt == 1) return pick_vec<DIM, F16, F16>(vec_bytes);
  if (vdt == 1 && cdt == 0) return pick_vec<DIM, F16, F32>(vec_bytes);
  if (vdt == 2 && cdt == 2) return pick_vec<DIM, BF16, BF16>(vec_bytes);
  if (vdt == 2 && cdt == 0) return pick_vec<DIM, BF16, F32>(vec_bytes);
  return nullptr;
}

LaunchFn get_fwd_launcher(int dim, int vdt, int cdt, int vec_bytes) {
  if (dim == 2) return pick_types<2>(vdt, cdt, vec_bytes);
  if (dim == 3) return pick_types<3>(vdt, cdt, vec_bytes);
  return nullptr;
}

}  // namespace msda
