// msda_fwd.hip — gfx950 forward kernels: bilinear (2D) / trilinear (3D) multi-scale
// deformable attention.
//
// Work decomposition. A "unit" is one (batch b, query q, head h), owned by an aligned
// group of 2^lpu_log2 lanes of one wave64. Lane j of the group holds channels
// [j*VEC, (j+1)*VEC), so each corner of a sample is one VEC*sizeof(value)-byte load per
// lane (16 B when C allows) and the group together reads one contiguous C-channel value
// row. Samples are processed in batches of SB: all SB*2^DIM corner loads of a batch are
// issued before any is consumed, which keeps 16 row loads in flight per lane. Accumulation
// is fp32 and the output is rounded once to the value dtype.
//
// Two kernels share that per-unit code:
//  * msda_fwd_kernel: units in (b, head-group, q, head-in-group) order so the heads that
//    share 128-byte lines of loc/attn/output run side by side; workgroups remapped so each
//    XCD owns a contiguous unit range and keeps a (batch, head-group) value slice in its
//    L2. Corners outside the level read as zero through the buffer range check.
//  * msda_fwd_staged_kernel: one 768-thread workgroup per CU serves one (batch, head) and
//    a range of queries. It first copies the smallest levels of that (batch, head) value
//    slice that fit kFwdStageLds into LDS; corners on those levels are then read from LDS,
//    the others from L2 (their slices again XCD-resident). Every row gather goes to L2 as a
//    full 128-byte line of which one head uses 64 bytes, so serving the coarse levels from
//    LDS removes their share of the L2 line traffic, which bounds this kernel.
#include "msda_internal.h"
#include "msda_sample.h"

namespace msda {

namespace {

struct Unit {
  uint32_t b, q, h, lane, bqh;
};

__device__ inline bool decode_unit(const Params& p, Unit& u) {
  const uint32_t lb = xcd_logical_block(blockIdx.x, p.nblocks, p.xcds);
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

// Per-level addressing of the forward. A corner row (x, y, z) of a level is read at byte
// offset  unit base + base + z*sz + y*sy + x*sx  from the value slice (global levels, unit
// base = the unit's (b, h, lane) offset) or from the staged rows in LDS (unit base = the
// lane's offset in a row).
struct FwdLevel {
  int32_t start, W, H, D;  // first row in K and extents (D = 1 in 2D)
  uint32_t base;           // global: start * rs; staged: first LDS byte of the level
  int32_t sx, sy, sz;      // byte strides along x, y, z
  int32_t flags;           // kLvlStaged | kLvlMul24
  float inv[3];            // 1 / W, 1 / H, 1 / D (fused producer path)
};
constexpr int32_t kLvlStaged = 1;  // rows are in LDS
constexpr int32_t kLvlMul24 = 2;   // strides and extents fit 24-bit signed multiplies

// Strides of a level whose rows are sx bytes apart; kLvlMul24 when every stride used and
// every index in [-2, extent + 1] fits a signed 24-bit multiplier input.
template <int DIM>
__device__ inline void set_strides(FwdLevel& e, uint32_t sx) {
  const uint64_t sy = (uint64_t)e.W * sx, sz = sy * (uint64_t)e.H;
  constexpr uint64_t lim = 1u << 23;
  e.sx = (int32_t)sx;
  e.sy = (int32_t)sy;
  e.sz = DIM == 3 ? (int32_t)sz : 0;
  const uint64_t ext = (uint64_t)max(max(e.W, e.H), e.D) + 2;
  const bool m24 = sx < lim && sy < lim && (DIM == 2 || sz < lim) && ext < lim;
  e.flags = (e.flags & ~kLvlMul24) | (m24 ? kLvlMul24 : 0);
}

// Bytes between consecutive rows of K, and the first byte of the (b, h) slice, in the
// (B, K, H, C) value or its head-major (B, H, K, C) copy.
__device__ inline uint32_t row_stride(const Params& p, int eb) {
  return (p.value_h ? 1u : (uint32_t)p.H) * (uint32_t)p.C * (uint32_t)eb;
}
__device__ inline uint32_t slice_base(const Params& p, uint32_t b, uint32_t h, int eb) {
  return (p.value_h ? (b * (uint32_t)p.H + h) * (uint32_t)p.K : b * (uint32_t)p.K * (uint32_t)p.H + h) *
         (uint32_t)p.C * (uint32_t)eb;
}

// Level table for global reads with rows rs bytes apart.
template <int DIM>
__device__ inline void stage_levels(const Params& p, FwdLevel* s_lvl, uint32_t rs) {
  for (int i = threadIdx.x; i < p.L; i += blockDim.x) {
    FwdLevel e;
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
    e.base = (uint32_t)e.start * rs;
    e.flags = 0;
    e.inv[0] = 1.0f / (float)e.W;
    e.inv[1] = 1.0f / (float)e.H;
    e.inv[2] = 1.0f / (float)e.D;
    set_strides<DIM>(e, rs);
    s_lvl[i] = e;
  }
}

// Corner rows of a batch of samples: from the global value slice through the buffer range
// check (kOobOffset reads zero), or, for a level held in LDS, from its staged rows (invalid
// corners read the all-zero row at zoff). ubase is the unit's byte base (see FwdLevel).
// M24: the level's strides fit 24-bit multiplies (full-rate v_mad_i32_i24 instead of
// quarter-rate 32-bit multiplies).
template <int DIM, int VB, int SB, bool LDS, bool M24>
__device__ inline void fetch_rows(const Sample<DIM> (&sm)[SB], const FwdLevel& lv,
                                  __amdgpu_buffer_rsrc_t rv, uint32_t ubase, const char* s_rows,
                                  uint32_t zoff, RawVec<VB> (&raw)[SB][1 << DIM]) {
  constexpr int NC = 1 << DIM;
#pragma unroll
  for (int k = 0; k < SB; ++k) {
    int32_t o0;
    if constexpr (M24) {
      o0 = __mul24(sm[k].ay.i0, lv.sy) + __mul24(sm[k].ax.i0, lv.sx);
      if constexpr (DIM == 3) o0 += __mul24(sm[k].az.i0, lv.sz);
    } else {
      o0 = sm[k].ay.i0 * lv.sy + sm[k].ax.i0 * lv.sx;
      if constexpr (DIM == 3) o0 += sm[k].az.i0 * lv.sz;
    }
    const uint32_t o = ubase + lv.base + (uint32_t)o0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t dr = ((c & 1) ? (uint32_t)lv.sx : 0u) + ((c & 2) ? (uint32_t)lv.sy : 0u) +
                          ((DIM == 3 && (c & 4)) ? (uint32_t)lv.sz : 0u);
      const bool ok = corner_valid<DIM>(c, sm[k]);
      if constexpr (LDS)
        raw[k][c] = *reinterpret_cast<const RawVec<VB>*>(s_rows + (ok ? o + dr : zoff));
      else
        raw[k][c] = buf_load<VB>(rv, ok ? o + dr : kOobOffset);
    }
  }
}

// fetch_rows with the level's storage and multiplier chosen at run time (uniform branch).
template <int DIM, int VB, int SB, bool STAGED>
__device__ inline void fetch_level(const Sample<DIM> (&sm)[SB], const FwdLevel& lv,
                                   __amdgpu_buffer_rsrc_t rv, uint32_t vbase, uint32_t lane_off,
                                   const char* s_rows, uint32_t zoff, RawVec<VB> (&raw)[SB][1 << DIM]) {
  if (STAGED && (lv.flags & kLvlStaged)) {
    if (lv.flags & kLvlMul24) fetch_rows<DIM, VB, SB, true, true>(sm, lv, rv, lane_off, s_rows, zoff, raw);
    else fetch_rows<DIM, VB, SB, true, false>(sm, lv, rv, lane_off, s_rows, zoff, raw);
  } else {
    if (lv.flags & kLvlMul24) fetch_rows<DIM, VB, SB, false, true>(sm, lv, rv, vbase, s_rows, zoff, raw);
    else fetch_rows<DIM, VB, SB, false, false>(sm, lv, rv, vbase, s_rows, zoff, raw);
  }
}

// The whole forward of one unit: sum over levels and points of attn * sample(value).
//
// PT > 0: the number of points per level is a compile-time constant; every coordinate and
// weight block of the unit is loaded before its first row gather, and all corner rows of a
// batch are issued before any is consumed. Used when the unit's blocks fit kFwdCoordSlots<DIM>
// per lane (L * P / SB <= kFwdCoordSlots * nvec). PT == 0 handles any P with per-sample
// loads.
//
// STAGED: levels flagged kLvlStaged are read from s_rows; zoff is the lane's offset in the
// all-zero row there.
//
// SHARE (PT > 0, units of 4, 8, ... lanes, all active): lane q of each quad computes the
// geometry of sample q % SB of the batch only (corner weights times attn, and corner row
// offsets without its own channel offset); the quad's lanes exchange those with DPP
// quad broadcasts instead of each lane recomputing every sample of the batch.
template <int K>
__device__ inline uint32_t quad_bcast(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, K * 0x55, 0xF, 0xF, true);
}

// Value x of lane j of the unit's lane group (first lane gbase), for j < nvec.
__device__ inline float group_lane(int gbase, int j, float x) {
  return as_float((uint32_t)__builtin_amdgcn_ds_bpermute((gbase + j) << 2, (int)as_u32(x)));
}

// Fused producer path: the unit's offset and logit blocks are held like location and weight
// blocks (coord dtype EC); each sample's location and weight are formed when its batch is
// used:
//   loc[d] = fma(off[d], 1 / size_l[d], ref[l][d]),   size_l = (W, H[, D]) of its level l
//   attn   = exp(logit - max) * (1 / sum exp(logit - max))   over the unit's L*P logits
// FusedStats holds the unit's max and 1/sum, reduced over its lanes in lane order (so every
// lane of the unit uses the same two values), and lane j's copy of the reference point of
// level j (used when L <= nvec; otherwise the reference points are read per batch).
template <int DIM>
struct FusedStats {
  float m, inv_sum;
  float ref[DIM];
};

template <int DIM, typename EC, int SB, int NS>
__device__ inline FusedStats<DIM> fused_stats(const Params& p, uint32_t bq, uint32_t lane,
                                              int nbatch, int gbase,
                                              const CoordBlock<EC, SB> (&ha)[NS]) {
  const int nv = p.nvec;
  FusedStats<DIM> st;
  float mx = -INFINITY;
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
    if ((int)lane + sl * nv < nbatch)
#pragma unroll
      for (int k = 0; k < SB; ++k) mx = fmaxf(mx, block_elem(ha[sl], k));
  st.m = -INFINITY;
  for (int j = 0; j < nv; ++j) st.m = fmaxf(st.m, group_lane(gbase, j, mx));
  float ls = 0.0f;
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
    if ((int)lane + sl * nv < nbatch)
#pragma unroll
      for (int k = 0; k < SB; ++k) ls += expf(block_elem(ha[sl], k) - st.m);
  float sum = 0.0f;
  for (int j = 0; j < nv; ++j) sum += group_lane(gbase, j, ls);
  st.inv_sum = 1.0f / sum;
  const float* refp = p.ref + (size_t)bq * (uint32_t)(p.L * DIM);
#pragma unroll
  for (int d = 0; d < DIM; ++d) st.ref[d] = (int)lane < p.L ? refp[lane * DIM + d] : 0.0f;
  return st;
}

// Reference point of level l for the unit (uniform l): from lane l of the group, or from
// memory when the levels outnumber the lanes.
template <int DIM>
__device__ inline void fused_ref(const Params& p, const FusedStats<DIM>& st, uint32_t bq, int gbase,
                                 int l, float (&r)[DIM]) {
  if (p.L <= p.nvec) {
#pragma unroll
    for (int d = 0; d < DIM; ++d) r[d] = group_lane(gbase, l, st.ref[d]);
  } else {
    const float* refp = p.ref + (size_t)bq * (uint32_t)(p.L * DIM) + l * DIM;
#pragma unroll
    for (int d = 0; d < DIM; ++d) r[d] = refp[d];
  }
}

// FUSED: p.loc / p.attn hold offsets and logits and p.ref the reference points (see
// Params); bq = b * Q + q indexes the unit's reference points.
template <int DIM, typename EV, typename EC, int VEC, int PT, bool STAGED, bool SHARE = false,
          bool FUSED = false>
__device__ inline void unit_forward(const Params& p, const FwdLevel* s_lvl, const char* s_rows,
                                    uint32_t zoff, uint32_t b, uint32_t h, uint32_t bqh,
                                    uint32_t bq, uint32_t lane, float (&acc)[VEC]) {
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  constexpr int SB = PT > 0 ? (DIM == 2 ? (PT < 4 ? PT : 4) : (PT < 2 ? PT : 2)) : (DIM == 2 ? 4 : 2);
  typedef typename EC::T TC;
  const int LP = p.L * p.P;
  const TC* locp = static_cast<const TC*>(p.loc) + (size_t)bqh * (LP * DIM);
  const TC* attp = static_cast<const TC*>(p.attn) + (size_t)bqh * LP;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.value_h ? p.value_h : p.value, p.value_bytes);
  const uint32_t lane_off = lane * VB;
  const uint32_t vbase = slice_base(p, b, h, EV::kBytes) + lane_off;

#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;

  if constexpr (PT > 0) {
    // The unit's coordinate and weight blocks (one per batch of SB samples) are fetched
    // up front, spread over its lanes: lane j holds batches j, j + nvec, ... With one
    // independent load per lane and slot, no batch waits on a coordinate load; each batch
    // broadcasts its block from the holding lane (ds_bpermute within the lane group).
    constexpr int BPL = PT / SB;  // batches per level
    constexpr int LW = CoordBlock<EC, SB * DIM>::kDwords, AW = CoordBlock<EC, SB>::kDwords;
    const int nbatch = p.L * BPL;
    const int nv = p.nvec;
    CoordBlock<EC, SB * DIM> hl[kFwdCoordSlots<DIM>];
    CoordBlock<EC, SB> ha[kFwdCoordSlots<DIM>];
    const int gbase = (int)(__lane_id() & ~((1u << p.lpu_log2) - 1u));  // first lane of the group
#pragma unroll
    for (int sl = 0; sl < kFwdCoordSlots<DIM>; ++sl) {
      const int bj = (int)lane + sl * nv;
      if (bj < nbatch) {
        load_block<EC, SB * DIM>(hl[sl], locp + bj * (SB * DIM));
        load_block<EC, SB>(ha[sl], attp + bj * SB);
      }
    }
    FusedStats<DIM> fst;
    if constexpr (FUSED) fst = fused_stats<DIM, EC, SB, kFwdCoordSlots<DIM>>(p, bq, lane, nbatch, gbase, ha);
    if constexpr (SHARE) {
      const int ks = (int)(lane & 3u) % SB;  // the batch sample this lane computes
      const uint32_t vbase0 = vbase - lane_off;
      const uint32_t zoff0 = zoff - lane_off;
#pragma unroll 1
      for (int bi = 0; bi < nbatch; ++bi) {
        const int l = bi / BPL;
        const FwdLevel lv = s_lvl[l];
        const int sl = bi / nv;
        const int src = (gbase + (bi - sl * nv)) << 2;
        CoordBlock<EC, SB * DIM> lb;
        CoordBlock<EC, SB> ab;
#pragma unroll
        for (int w = 0; w < LW; ++w) {
          uint32_t x = hl[0].d[w];
#pragma unroll
          for (int k = 1; k < kFwdCoordSlots<DIM>; ++k) x = sl == k ? hl[k].d[w] : x;
          lb.d[w] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)x);
        }
#pragma unroll
        for (int w = 0; w < AW; ++w) {
          uint32_t x = ha[0].d[w];
#pragma unroll
          for (int k = 1; k < kFwdCoordSlots<DIM>; ++k) x = sl == k ? ha[k].d[w] : x;
          ab.d[w] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)x);
        }
        // this lane's sample: coordinates and weight picked from the batch block
        float xyz[DIM], a = block_elem(ab, 0);
#pragma unroll
        for (int d = 0; d < DIM; ++d) xyz[d] = block_elem(lb, d);
#pragma unroll
        for (int k = 1; k < SB; ++k) {
          a = ks == k ? block_elem(ab, k) : a;
#pragma unroll
          for (int d = 0; d < DIM; ++d) xyz[d] = ks == k ? block_elem(lb, k * DIM + d) : xyz[d];
        }
        if constexpr (FUSED) {
          float r[DIM];
          fused_ref<DIM>(p, fst, bq, gbase, l, r);
#pragma unroll
          for (int d = 0; d < DIM; ++d) xyz[d] = __builtin_fmaf(xyz[d], lv.inv[d], r[d]);
          a = expf(a - fst.m) * fst.inv_sum;
        }
        Sample<DIM> sm;
        sm.ax = make_axis(xyz[0], (float)lv.W, lv.W, p.clamp, p.lo_g, p.hi_g);
        sm.ay = make_axis(xyz[1], (float)lv.H, lv.H, p.clamp, p.lo_g, p.hi_g);
        if constexpr (DIM == 3) sm.az = make_axis(xyz[2], (float)lv.D, lv.D, p.clamp, p.lo_g, p.hi_g);
        const bool lds = STAGED && (lv.flags & kLvlStaged);
        int32_t o0;
        if (lv.flags & kLvlMul24) {
          o0 = __mul24(sm.ay.i0, lv.sy) + __mul24(sm.ax.i0, lv.sx);
          if constexpr (DIM == 3) o0 += __mul24(sm.az.i0, lv.sz);
        } else {
          o0 = sm.ay.i0 * lv.sy + sm.ax.i0 * lv.sx;
          if constexpr (DIM == 3) o0 += sm.az.i0 * lv.sz;
        }
        const uint32_t obase = (lds ? 0u : vbase0) + lv.base + (uint32_t)o0;
        const uint32_t obad = lds ? zoff0 : kOobOffset;
        uint32_t mo[NC], mw[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const uint32_t dr = ((c & 1) ? (uint32_t)lv.sx : 0u) + ((c & 2) ? (uint32_t)lv.sy : 0u) +
                              ((DIM == 3 && (c & 4)) ? (uint32_t)lv.sz : 0u);
          mo[c] = corner_valid<DIM>(c, sm) ? obase + dr : obad;
          mw[c] = as_u32(corner_weight<DIM>(c, sm) * a);
        }
        // every sample of the batch from the quad lane that computed it
        uint32_t off[SB][NC];
        float cw[SB][NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          off[0][c] = quad_bcast<0>(mo[c]) + lane_off;
          cw[0][c] = as_float(quad_bcast<0>(mw[c]));
          if constexpr (SB > 1) {
            off[1][c] = quad_bcast<1>(mo[c]) + lane_off;
            cw[1][c] = as_float(quad_bcast<1>(mw[c]));
          }
          if constexpr (SB > 2) {
            off[2][c] = quad_bcast<2>(mo[c]) + lane_off;
            cw[2][c] = as_float(quad_bcast<2>(mw[c]));
          }
          if constexpr (SB > 3) {
            off[3][c] = quad_bcast<3>(mo[c]) + lane_off;
            cw[3][c] = as_float(quad_bcast<3>(mw[c]));
          }
        }
        RawVec<VB> raw[SB][NC];
        if (lds) {
#pragma unroll
          for (int k = 0; k < SB; ++k)
#pragma unroll
            for (int c = 0; c < NC; ++c) raw[k][c] = *reinterpret_cast<const RawVec<VB>*>(s_rows + off[k][c]);
        } else {
#pragma unroll
          for (int k = 0; k < SB; ++k)
#pragma unroll
            for (int c = 0; c < NC; ++c) raw[k][c] = buf_load<VB>(rv, off[k][c]);
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
      return;
    }
#pragma unroll 1
    for (int bi = 0; bi < nbatch; ++bi) {
      const int l = bi / BPL;
      const FwdLevel lv = s_lvl[l];
      const int sl = bi / nv;
      const int src = (gbase + (bi - sl * nv)) << 2;
      CoordBlock<EC, SB * DIM> lb;
      CoordBlock<EC, SB> ab;
#pragma unroll
      for (int w = 0; w < LW; ++w) {
        uint32_t x = hl[0].d[w];
#pragma unroll
        for (int k = 1; k < kFwdCoordSlots<DIM>; ++k) x = sl == k ? hl[k].d[w] : x;
        lb.d[w] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)x);
      }
#pragma unroll
      for (int w = 0; w < AW; ++w) {
        uint32_t x = ha[0].d[w];
#pragma unroll
        for (int k = 1; k < kFwdCoordSlots<DIM>; ++k) x = sl == k ? ha[k].d[w] : x;
        ab.d[w] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)x);
      }
      Sample<DIM> sm[SB];
      float cw[SB][NC];
      float r[DIM];
      if constexpr (FUSED) fused_ref<DIM>(p, fst, bq, gbase, l, r);
#pragma unroll
      for (int k = 0; k < SB; ++k) {
        float xyz[DIM], a = block_elem(ab, k);
#pragma unroll
        for (int d = 0; d < DIM; ++d) xyz[d] = block_elem(lb, k * DIM + d);
        if constexpr (FUSED) {
#pragma unroll
          for (int d = 0; d < DIM; ++d) xyz[d] = __builtin_fmaf(xyz[d], lv.inv[d], r[d]);
          a = expf(a - fst.m) * fst.inv_sum;
        }
        sm[k].ax = make_axis(xyz[0], (float)lv.W, lv.W, p.clamp, p.lo_g, p.hi_g);
        sm[k].ay = make_axis(xyz[1], (float)lv.H, lv.H, p.clamp, p.lo_g, p.hi_g);
        if constexpr (DIM == 3) sm[k].az = make_axis(xyz[2], (float)lv.D, lv.D, p.clamp, p.lo_g, p.hi_g);
#pragma unroll
        for (int c = 0; c < NC; ++c) cw[k][c] = corner_weight<DIM>(c, sm[k]) * a;
      }
      RawVec<VB> raw[SB][NC];
      fetch_level<DIM, VB, SB, STAGED>(sm, lv, rv, vbase, lane_off, s_rows, zoff, raw);
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
    // FUSED: softmax statistics of the unit's logits, each lane over all of them
    float smax = 0.0f, inv_sum = 1.0f;
    if constexpr (FUSED) {
      smax = -INFINITY;
      for (int s = 0; s < LP; ++s) smax = fmaxf(smax, (float)attp[s]);
      float ssum = 0.0f;
      for (int s = 0; s < LP; ++s) ssum += expf((float)attp[s] - smax);
      inv_sum = 1.0f / ssum;
    }
    const float* refp = FUSED ? p.ref + (size_t)bq * (uint32_t)(p.L * DIM) : nullptr;
    for (int l = 0; l < p.L; ++l) {
      const FwdLevel lv = s_lvl[l];
      for (int p0 = 0; p0 < p.P; p0 += SB) {
        Sample<DIM> sm[SB];
        float cw[SB][NC];
#pragma unroll
        for (int k = 0; k < SB; ++k) {
          const int s = l * p.P + p0 + k;
          const bool live = p0 + k < p.P;
          const TC* lp = locp + (live ? s : 0) * DIM;
          float a, xyz[DIM];
          if constexpr (FUSED) {
            a = live ? expf((float)attp[s] - smax) * inv_sum : 0.0f;
#pragma unroll
            for (int d = 0; d < DIM; ++d) xyz[d] = __builtin_fmaf((float)lp[d], lv.inv[d], refp[l * DIM + d]);
          } else {
            a = live ? (float)attp[s] : 0.0f;
#pragma unroll
            for (int d = 0; d < DIM; ++d) xyz[d] = (float)lp[d];
          }
          sm[k].ax = make_axis(xyz[0], (float)lv.W, lv.W, p.clamp, p.lo_g, p.hi_g);
          sm[k].ay = make_axis(xyz[1], (float)lv.H, lv.H, p.clamp, p.lo_g, p.hi_g);
          if constexpr (DIM == 3) sm[k].az = make_axis(xyz[2], (float)lv.D, lv.D, p.clamp, p.lo_g, p.hi_g);
#pragma unroll
          for (int c = 0; c < NC; ++c) cw[k][c] = corner_weight<DIM>(c, sm[k]) * a;
        }
        RawVec<VB> raw[SB][NC];
        fetch_level<DIM, VB, SB, STAGED>(sm, lv, rv, vbase, lane_off, s_rows, zoff, raw);
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
}

}  // namespace

// Replaces the reference's _fwd_kernel_2d (src/msda_triton/triton/msda_2d.py:85-260) and
// _fwd_kernel (src/msda_triton/triton/msda_3d.py:80-288). Writes (B, Q, H*C) in the value
// dtype directly instead of an fp32 (B*H, Q, C) scratch plus permute (msda_2d.py:649-651).
template <int DIM, typename EV, typename EC, int VEC, int PT, bool FUSED>
__global__ __launch_bounds__(kBlock) void msda_fwd_kernel(const Params p) {
  __shared__ FwdLevel s_lvl[kMaxLevels];
  stage_levels<DIM>(p, s_lvl, row_stride(p, EV::kBytes));
  __syncthreads();
  Unit u;
  if (!decode_unit(p, u)) return;
  if ((int)u.lane >= p.nvec) return;
  float acc[VEC];
  unit_forward<DIM, EV, EC, VEC, PT, false, false, FUSED>(p, s_lvl, nullptr, 0u, u.b, u.h, u.bqh,
                                                         u.b * p.Q + u.q, u.lane, acc);
  typename EV::T* outp = static_cast<typename EV::T*>(p.out) + (size_t)u.bqh * p.C + u.lane * VEC;
  store_vec<EV, VEC>(outp, acc);
}

// Same result as msda_fwd_kernel; the smallest levels of the workgroup's (batch, head)
// value slice are read from LDS.
template <int DIM, typename EV, typename EC, int VEC, int PT, bool SHARE, bool FUSED>
__global__ __launch_bounds__(kFwdStageThreads) void msda_fwd_staged_kernel(const Params p) {
  constexpr int NT = kFwdStageThreads;
  constexpr int VB = VEC * EV::kBytes;
  extern __shared__ __attribute__((aligned(16))) char s_rows[];
  __shared__ FwdLevel s_lvl[kMaxLevels];
  __shared__ int32_t s_order[kMaxLevels];  // staged levels in LDS order
  __shared__ uint32_t s_pfx[kMaxLevels + 1];  // their first piece in the flat staging index
  __shared__ int32_t s_nst;
  const uint32_t lrs = (uint32_t)p.C * EV::kBytes;  // bytes per staged row
  stage_levels<DIM>(p, s_lvl, row_stride(p, EV::kBytes));
  __syncthreads();
  const uint32_t nvec = (uint32_t)p.nvec;
  if (threadIdx.x == 0) {
    // greedy: smallest levels first, while they fit beside the all-zero row
    const uint32_t cap = p.stage_bytes / lrs - 1u;  // the host guarantees >= 2 rows
    uint32_t used = 0;
    int n = 0;
    for (;;) {
      int best = -1;
      uint32_t bsz = 0;
      for (int l = 0; l < p.L; ++l) {
        if (s_lvl[l].flags & kLvlStaged) continue;
        const uint32_t sz = (uint32_t)s_lvl[l].W * (uint32_t)s_lvl[l].H * (uint32_t)s_lvl[l].D;
        if (sz == 0 || used + sz > cap) continue;
        if (best < 0 || sz < bsz) {
          best = l;
          bsz = sz;
        }
      }
      if (best < 0) break;
      FwdLevel& e = s_lvl[best];
      e.flags |= kLvlStaged;
      e.base = used * lrs;
      set_strides<DIM>(e, lrs);
      s_order[n] = best;
      s_pfx[n] = used * nvec;
      used += bsz;
      ++n;
    }
    s_pfx[n] = used * nvec;
    s_nst = n;
  }
  __syncthreads();
  const uint32_t zrow = s_pfx[s_nst] / nvec * lrs;  // byte offset of the all-zero row

  const uint32_t lb = xcd_logical_block(blockIdx.x, p.nblocks, p.xcds);
  const uint32_t bh = lb / p.splits, split = lb - bh * p.splits;
  const uint32_t b = bh / (uint32_t)p.H, h = bh - b * (uint32_t)p.H;
  const uint32_t q0 = split * p.qper;
  const uint32_t q1 = min(p.Q, q0 + p.qper);

  // copy the staged levels' rows of (b, h): every load of a thread is issued before any of
  // its stores
  {
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.value_h ? p.value_h : p.value, p.value_bytes);
    const uint32_t rs = row_stride(p, EV::kBytes);
    const uint32_t vrow0 = slice_base(p, b, h, EV::kBytes);
    const int nst = s_nst;
    const uint32_t total = s_pfx[nst];
    constexpr int KB = 8;
    for (uint32_t i0 = threadIdx.x; i0 < total; i0 += KB * NT) {
      RawVec<VB> v[KB];
      uint32_t dst[KB];
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        const uint32_t i = i0 + (uint32_t)k * NT;
        uint32_t goff = kOobOffset;
        dst[k] = 0xffffffffu;
        if (i < total) {
          int j = 0;
          while (j + 1 < nst && s_pfx[j + 1] <= i) ++j;
          const uint32_t rel = i - s_pfx[j];
          const uint32_t r = rel / nvec, ch = rel - r * nvec;
          const int l = s_order[j];
          goff = vrow0 + ((uint32_t)s_lvl[l].start + r) * rs + ch * VB;
          dst[k] = s_lvl[l].base + r * lrs + ch * VB;
        }
        v[k] = buf_load<VB>(rv, goff);
      }
#pragma unroll
      for (int k = 0; k < KB; ++k)
        if (dst[k] != 0xffffffffu) *reinterpret_cast<RawVec<VB>*>(s_rows + dst[k]) = v[k];
    }
    if (threadIdx.x < nvec) *reinterpret_cast<RawVec<VB>*>(s_rows + zrow + threadIdx.x * VB) = RawVec<VB>{};
  }
  __syncthreads();

  const uint32_t lanes_log2 = (uint32_t)p.lpu_log2;
  const uint32_t lane = threadIdx.x & ((1u << lanes_log2) - 1u);
  const uint32_t upi = (uint32_t)NT >> lanes_log2;  // units per iteration
  if ((int)lane >= p.nvec) return;  // no barrier follows
  for (uint32_t qb = q0; qb < q1; qb += upi) {
    const uint32_t q = qb + (threadIdx.x >> lanes_log2);
    if (q >= q1) break;
    const uint32_t bqh = (b * p.Q + q) * (uint32_t)p.H + h;
    float acc[VEC];
    unit_forward<DIM, EV, EC, VEC, PT, true, SHARE, FUSED>(p, s_lvl, s_rows, zrow + lane * VB, b, h, bqh,
                                                           b * p.Q + q, lane, acc);
    typename EV::T* outp = static_cast<typename EV::T*>(p.out) + (size_t)bqh * p.C + lane * VEC;
    store_vec<EV, VEC>(outp, acc);
  }
}

// The compile-time point counts (4 and 8 points per level) need aligned coordinate blocks
// and a unit's blocks within kFwdCoordSlots per lane.
template <int DIM, int PT>
static bool pt_path(const Params& p) {
  constexpr int SB = DIM == 2 ? (PT < 4 ? PT : 4) : (PT < 2 ? PT : 2);
  return p.P == PT && p.coords_aligned && p.L * (PT / SB) <= kFwdCoordSlots<DIM> * p.nvec;
}

template <int DIM, typename EV, typename EC, int VEC, bool FUSED>
static hipError_t launch_fwd(const Params& p, hipStream_t s) {
  if (pt_path<DIM, 4>(p))
    hipLaunchKernelGGL((msda_fwd_kernel<DIM, EV, EC, VEC, 4, FUSED>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  else if (pt_path<DIM, 8>(p))
    hipLaunchKernelGGL((msda_fwd_kernel<DIM, EV, EC, VEC, 8, FUSED>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  else
    hipLaunchKernelGGL((msda_fwd_kernel<DIM, EV, EC, VEC, 0, FUSED>), dim3(p.nblocks), dim3(kBlock), 0, s, p);
  return hipGetLastError();
}

template <int DIM, typename EV, typename EC, int VEC, bool FUSED>
static hipError_t launch_fwd_staged(const Params& p, hipStream_t s) {
  const dim3 g(p.nblocks), t(kFwdStageThreads);
  // quad-shared geometry when every lane of a unit's 4-lane quads is active
  const bool share = p.lpu_log2 >= 2 && p.nvec == (1 << p.lpu_log2);
  if (pt_path<DIM, 4>(p) && share)
    hipLaunchKernelGGL((msda_fwd_staged_kernel<DIM, EV, EC, VEC, 4, true, FUSED>), g, t, p.stage_bytes, s, p);
  else if (pt_path<DIM, 8>(p) && share)
    hipLaunchKernelGGL((msda_fwd_staged_kernel<DIM, EV, EC, VEC, 8, true, FUSED>), g, t, p.stage_bytes, s, p);
  else if (pt_path<DIM, 4>(p))
    hipLaunchKernelGGL((msda_fwd_staged_kernel<DIM, EV, EC, VEC, 4, false, FUSED>), g, t, p.stage_bytes, s, p);
  else if (pt_path<DIM, 8>(p))
    hipLaunchKernelGGL((msda_fwd_staged_kernel<DIM, EV, EC, VEC, 8, false, FUSED>), g, t, p.stage_bytes, s, p);
  else
    hipLaunchKernelGGL((msda_fwd_staged_kernel<DIM, EV, EC, VEC, 0, false, FUSED>), g, t, p.stage_bytes, s, p);
  return hipGetLastError();
}

template <int DIM, typename EV, typename EC, bool FUSED>
static LaunchFn pick_vec(int vec_bytes, bool staged) {
  constexpr int S = EV::kBytes;
  switch (vec_bytes) {
    case 16: return staged ? &launch_fwd_staged<DIM, EV, EC, 16 / S, FUSED> : &launch_fwd<DIM, EV, EC, 16 / S, FUSED>;
    case 8: return staged ? &launch_fwd_staged<DIM, EV, EC, 8 / S, FUSED> : &launch_fwd<DIM, EV, EC, 8 / S, FUSED>;
    case 4: return staged ? &launch_fwd_staged<DIM, EV, EC, 4 / S, FUSED> : &launch_fwd<DIM, EV, EC, 4 / S, FUSED>;
    case 2:
      if constexpr (S == 2) return staged ? &launch_fwd_staged<DIM, EV, EC, 1, FUSED> : &launch_fwd<DIM, EV, EC, 1, FUSED>;
      return nullptr;
    default: return nullptr;
  }
}

template <int DIM, bool FUSED>
static LaunchFn pick_types(int vdt, int cdt, int vec_bytes, bool staged) {
  if (vdt == 0 && cdt == 0) return pick_vec<DIM, F32, F32, FUSED>(vec_bytes, staged);
  if (vdt == 1 && cdt == 1) return pick_vec<DIM, F16, F16, FUSED>(vec_bytes, staged);
  if (vdt == 1 && cdt == 0) return pick_vec<DIM, F16, F32, FUSED>(vec_bytes, staged);
  if (vdt == 2 && cdt == 2) return pick_vec<DIM, BF16, BF16, FUSED>(vec_bytes, staged);
  if (vdt == 2 && cdt == 0) return pick_vec<DIM, BF16, F32, FUSED>(vec_bytes, staged);
  return nullptr;
}

// Head-major copy: thread i moves chunk i of value in (b, k, h, chunk) order, so reads are
// contiguous and the 2 keys x H heads of a wave write whole 128-byte lines per head.
template <int VB>
__global__ __launch_bounds__(kBlock) void head_major_kernel(const char* __restrict__ src,
                                                           char* __restrict__ dst, uint32_t n,
                                                           FastDiv div_c, FastDiv div_hc,
                                                           FastDiv div_khc, uint32_t K,
                                                           uint32_t H, uint32_t row) {
  const uint32_t stride = gridDim.x * kBlock;
  for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const uint32_t b = fdiv(i, div_khc), r0 = i - b * div_khc.d;
    const uint32_t k = fdiv(r0, div_hc), r1 = r0 - k * div_hc.d;
    const uint32_t h = fdiv(r1, div_c), c = r1 - h * div_c.d;
    const RawVec<VB> v = *reinterpret_cast<const RawVec<VB>*>(src + (size_t)i * VB);
    *reinterpret_cast<RawVec<VB>*>(dst + ((size_t)(b * H + h) * K + k) * row + (size_t)c * VB) = v;
  }
}

hipError_t launch_head_major(const void* src, void* dst, uint32_t B, uint32_t K, uint32_t H,
                             uint32_t row_bytes, int vec_bytes, hipStream_t s) {
  const uint32_t cpr = row_bytes / (uint32_t)vec_bytes;  // chunks per row
  const uint64_t n = (uint64_t)B * K * H * cpr;
  if (n == 0) return hipSuccess;
  const FastDiv dc = make_fastdiv(cpr), dhc = make_fastdiv(H * cpr), dkhc = make_fastdiv(K * H * cpr);
  const uint32_t blocks = (uint32_t)((n + kBlock - 1) / kBlock < 8192 ? (n + kBlock - 1) / kBlock : 8192);
  const char* sp = static_cast<const char*>(src);
  char* dp = static_cast<char*>(dst);
  switch (vec_bytes) {
    case 16: hipLaunchKernelGGL(head_major_kernel<16>, dim3(blocks), dim3(kBlock), 0, s, sp, dp, (uint32_t)n, dc, dhc, dkhc, K, H, row_bytes); break;
    case 8: hipLaunchKernelGGL(head_major_kernel<8>, dim3(blocks), dim3(kBlock), 0, s, sp, dp, (uint32_t)n, dc, dhc, dkhc, K, H, row_bytes); break;
    case 4: hipLaunchKernelGGL(head_major_kernel<4>, dim3(blocks), dim3(kBlock), 0, s, sp, dp, (uint32_t)n, dc, dhc, dkhc, K, H, row_bytes); break;
    case 2: hipLaunchKernelGGL(head_major_kernel<2>, dim3(blocks), dim3(kBlock), 0, s, sp, dp, (uint32_t)n, dc, dhc, dkhc, K, H, row_bytes); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

LaunchFn get_fwd_launcher(int dim, int vdt, int cdt, int vec_bytes, bool staged, bool fused) {
  if (dim == 2) return fused ? pick_types<2, true>(vdt, cdt, vec_bytes, staged) : pick_types<2, false>(vdt, cdt, vec_bytes, staged);
  if (dim == 3) return fused ? pick_types<3, true>(vdt, cdt, vec_bytes, staged) : pick_types<3, false>(vdt, cdt, vec_bytes, staged);
  return nullptr;
}

}  // namespace msda
