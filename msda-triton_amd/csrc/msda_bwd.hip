// msda_bwd.hip — gfx950 backward of multi-scale deformable attention without global
// floating-point atomics.
//
// Replaces the reference's _bwd_kernel_2d (src/msda_triton/triton/msda_2d.py:263-510) and
// 3D _bwd_kernel (src/msda_triton/triton/msda_3d.py:291-653), which scatter grad_value
// with one global atomic per (sample, corner, channel). On MI355X global fp32 atomics on
// random rows sustain about 0.33 T element-adds/s and LDS fp32 atomics about a third of
// an operation per clock per CU, so this backward accumulates grad_value in key order:
//
//  1. count: every sample with a valid corner is assigned, from its coordinates alone, to
//     the tile of its level that owns its lowest corner; each workgroup (upw units of one
//     (batch, head-group)) histograms its samples per tile in LDS (integer atomics, full
//     rate) and writes the histogram as one column of a tile-major (tile, workgroup)
//     count matrix.
//  2. column scan (one wave per tile): the tile's counts over the workgroups become
//     offsets within the tile, and the tile's total.
//  3. plan (one workgroup): exclusive scan of the tile totals, chunks of at most R records
//     per tile, and the chunk -> tile table.
//  4. fill: each workgroup ranks its samples per tile in LDS, sorts their records (id,
//     clamp flags, pixel coordinates, attention weight) by tile in LDS and writes them out
//     as contiguous runs.
//  5. tile kernel: one workgroup per chunk, chunks of one (batch, head-group) on one XCD.
//     It stages the value rows of the tile's region (the tile plus a one-cell high-side
//     halo, which holds every corner of a sample anchored in the tile) in LDS once. Per
//     sub-batch of S records it stages the records and their grad_out rows, forms each
//     record's corner dot products <grad_out, v_c> from LDS and stores the sample's
//     grad_attention_weights and clamp-masked grad_sampling_locations, sorts the
//     (corner weight * attn, record) entries by region cell (ranks come from the counting
//     atomics), and accumulates grad_value for every region cell in the fp32 registers of
//     the cell's owner threads. Interior cells of a one-chunk tile are written directly in
//     the value dtype; edge cells (which also receive halo contributions of lower
//     neighbours), halo cells and every cell of a split tile are written as fp32 partials.
//  6. fold: per tile, sums the partials of its own chunks and the halo partials of its
//     lower neighbours' chunks, in a fixed order, and writes the edge / split cells.
//
// Gathering the corner rows per sample (in query order, from L2) cost more than staging
// each tile's rows once: C2 bf16 sample gradients 106 us against an 11 us count pass plus
// 80 us more in the tile kernel; C5 350 us against 27 + 260 us.
//
// Every grad_value element is written exactly once with a plain store, so no clearing
// pass is needed and 16-bit values are rounded once, from fp32.
//
// Pyramids beyond the LDS binning (more than kMaxBinsLds tiles per head) and launches whose
// Q * P exceeds a record's 27-bit sample id instead gather each sample's corner rows per
// unit and scatter grad_value with global fp32 atomics into fp32 sums in the workspace,
// then round them in one pass.
#include "msda_internal.h"
#include "msda_sample.h"

namespace msda {

namespace {

constexpr int kPlanThreads = 1024;

// The launch's level geometry, read through the constant address space: the kernels never
// write it, so wave-uniform fields become scalar loads.
typedef const __attribute__((address_space(4))) BwdGeom* GeoP;

__device__ inline GeoP geo_of(const BwdBuffers& bf) { return (GeoP)bf.geom; }

__device__ inline BwdLevel level_at(GeoP g, int l) {
  BwdLevel lv;
  __builtin_memcpy(&lv, &g->lv[l], sizeof(BwdLevel));
  return lv;
}

// ------------------------------------------------------------------ block scans
// Inclusive scan across the 64 lanes of a wave with DPP: Hillis-Steele within each row of
// 16 lanes (row_shr 1, 2, 4, 8; lanes shifted in from outside the row read 0), then lane 15's
// sum added to rows 1 and 3 (row_bcast:15) and lane 31's to rows 2 and 3 (row_bcast:31).
// No LDS round trip (the ds_bpermute ladder it replaces cost six). Every lane of the wave
// must be active.
__device__ inline uint32_t wave_incl_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);   // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);   // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);   // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);   // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// Exclusive scan of one value per thread across a workgroup of NT threads; *total gets
// the sum. s_w holds NT / 64 words. Every thread of the workgroup must call it.
template <int NT>
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* s_w, uint32_t* total) {
  const uint32_t inc = wave_incl_scan(v);
  const int w = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  if (lane == kWave - 1) s_w[w] = inc;
  lds_sync();
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / kWave; ++i) {
    const uint32_t x = s_w[i];
    if (i < w) pre += x;
    tot += x;
  }
  lds_sync();
  *total = tot;
  return pre + inc - v;
}

// ------------------------------------------------------------------ tiles
struct TileCoord {
  uint32_t g, hsub, b, h;
  int l, tx, ty, tz, X0, Y0, Z0;
};

__device__ inline int level_of_tile(const BwdPlan& pl, GeoP geo, int tib) {
  int l = 0;
  while (l + 1 < pl.L && !(tib >= geo->lv[l].tile_off && tib < geo->lv[l].tile_off + geo->lv[l].ntiles)) ++l;
  return l;
}

__device__ inline TileCoord decode_tile(const BwdPlan& pl, GeoP geo, uint32_t t, BwdLevel* lvp) {
  TileCoord tc;
  const uint32_t bins = (uint32_t)geo->bins;
  tc.g = t / bins;
  const uint32_t bin = t - tc.g * bins;
  tc.hsub = bin & ((1u << pl.hg_log2) - 1u);
  const int tib = (int)(bin >> pl.hg_log2);
  const uint32_t gph = (uint32_t)pl.H >> pl.hg_log2;
  tc.b = tc.g / gph;
  tc.h = ((tc.g - tc.b * gph) << pl.hg_log2) | tc.hsub;
  tc.l = level_of_tile(pl, geo, tib);
  const BwdLevel lv = level_at(geo, tc.l);
  *lvp = lv;
  const int lt = tib - lv.tile_off;
  tc.tx = lt % lv.ntx;
  tc.ty = (lt / lv.ntx) % lv.nty;
  tc.tz = lt / (lv.ntx * lv.nty);
  tc.X0 = tc.tx * pl.TX;
  tc.Y0 = tc.ty * pl.TY;
  tc.Z0 = tc.tz * pl.TZ;
  return tc;
}

// The cells of a tile's region (the tile plus a one-cell high-side halo) that lie inside
// the level, numbered x fastest: a tile on the level's high edge has no halo there, and a
// partial tile only its own columns and rows. Corners never fall outside the level, so
// every cell of this compact region can receive entries.
struct Region {
  int ex, ey, ez;
};

__device__ inline Region tile_region(const BwdPlan& pl, const TileCoord& tc, const BwdLevel& lv) {
  Region rg;
  rg.ex = min(pl.RX, lv.W - tc.X0);
  rg.ey = min(pl.RY, lv.H - tc.Y0);
  rg.ez = min(pl.RZ, lv.D - tc.Z0);
  return rg;
}

// Compact region-cell index of a corner relative to the tile origin, or -1 outside.
__device__ inline int region_cell(const Region& rg, int ox, int oy, int oz) {
  if ((unsigned)ox >= (unsigned)rg.ex || (unsigned)oy >= (unsigned)rg.ey ||
      (unsigned)oz >= (unsigned)rg.ez)
    return -1;
  return (oz * rg.ey + oy) * rg.ex + ox;
}

// Region cell -> (x, y, z) offsets within the compact region. The quotients are formed as
// trunc((n + 0.5) * (1 / d)): for n < 2^20 the product's rounding error is below
// 2^-3 / d, while (n + 0.5) / d lies at least 0.5 / d from an integer, so the result is
// exact, in three instructions instead of a twenty-instruction integer division.
struct RegionSplit {
  float rxy, rx;  // 1 / (ex * ey), 1 / ex
  int exy, ex;
};

__device__ inline RegionSplit region_split(const Region& rg) {
  RegionSplit r;
  r.exy = rg.ex * rg.ey;
  r.ex = rg.ex;
  r.rxy = 1.0f / (float)r.exy;
  r.rx = 1.0f / (float)r.ex;
  return r;
}

__device__ inline void split_cell(const RegionSplit& r, int cell, int& rx, int& ry, int& rz) {
  rz = (int)(((float)cell + 0.5f) * r.rxy);
  const int rxy = cell - rz * r.exy;
  ry = (int)(((float)rxy + 0.5f) * r.rx);
  rx = rxy - ry * r.ex;
}

// Unit of a bin workgroup: the wi-th of the upw units of workgroup w of group g.
struct BinUnit {
  uint32_t q, hsub, b, h;
  size_t bqh;
};

__device__ inline BinUnit bin_unit(const BwdPlan& pl, uint32_t g, uint32_t w, uint32_t wi) {
  BinUnit bu;
  const uint32_t U = w * (uint32_t)pl.upw + wi;
  bu.q = U >> pl.hg_log2;
  bu.hsub = U & ((1u << pl.hg_log2) - 1u);
  const uint32_t gph = (uint32_t)pl.H >> pl.hg_log2;
  bu.b = g / gph;
  bu.h = ((g - bu.b * gph) << pl.hg_log2) | bu.hsub;
  bu.bqh = ((size_t)bu.b * pl.Q + bu.q) * pl.H + bu.h;
  return bu;
}

// Pixel coordinates, clamp flags and anchor tile of one sample at location xyz; false if
// the sample has no corner inside its level.
template <int DIM>
__device__ inline bool sample_tile(const BwdPlan& pl, const BwdLevel& lv, const float* xyz, float* u,
                                   uint32_t* flags, int* tib) {
  bool px, py, pz = true;
  u[0] = grid_to_u(xyz[0], (float)lv.W, pl.clamp, pl.lo_g, pl.hi_g, &px);
  u[1] = grid_to_u(xyz[1], (float)lv.H, pl.clamp, pl.lo_g, pl.hi_g, &py);
  u[2] = 0.0f;
  if constexpr (DIM == 3) u[2] = grid_to_u(xyz[2], (float)lv.D, pl.clamp, pl.lo_g, pl.hi_g, &pz);
  const Axis ax = axis_from_u(u[0], lv.W, px);
  const Axis ay = axis_from_u(u[1], lv.H, py);
  const Axis az = DIM == 3 ? axis_from_u(u[2], lv.D, pz) : Axis{1.0f, 0.0f, 0, true, false, true};
  if (!(ax.v0 || ax.v1) || !(ay.v0 || ay.v1) || !(az.v0 || az.v1)) return false;
  const int tx = anchor_tile(ax, pl.tx_log2), ty = anchor_tile(ay, pl.ty_log2);
  const int tz = DIM == 3 ? anchor_tile(az, pl.tz_log2) : 0;
  *tib = lv.tile_off + (tz * lv.nty + ty) * lv.ntx + tx;
  *flags = (px ? kRecPassX : 0u) | (py ? kRecPassY : 0u) | (pz ? kRecPassZ : 0u);
  return true;
}

// ------------------------------------------------------------------ atomic path
// Gradients of one sample from its gathered corner rows: <grad_out, v_c> per corner, then
// d/d(attn) and (clamp-masked) d/d(loc) summed over the unit's lanes, so every lane of
// the group holds them. out = {grad_attn, grad_loc x, y[, z]}.
template <int DIM, typename EV, int VEC, int NC = (1 << DIM)>
__device__ inline void sample_grads(const BwdLevel& lv, const Sample<DIM>& sm,
                                    const RawVec<VEC * EV::kBytes> (&raw)[NC],
                                    const RawVec<VEC * EV::kBytes>& graw, float a, int lg,
                                    float (&out)[DIM + 1]) {
  float dot[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float d = 0.0f;
    if constexpr (EV::kBytes == 2 && VEC >= 2) {
      // value and grad_out are both 16-bit: packed dot products, exact products
#pragma unroll
      for (int e = 0; e < VEC / 2; ++e) d = dot2_acc<EV>(raw_dword(raw[c], e), raw_dword(graw, e), d);
    } else {
      float v[VEC], g[VEC];
      widen<EV, VEC>(raw[c], v);
      widen<EV, VEC>(graw, g);
#pragma unroll
      for (int e = 0; e < VEC; ++e) d = __builtin_fmaf(g[e], v[e], d);
    }
    dot[c] = d;
  }
  float s_attn, s_x, s_y, s_z;
  corner_grads<DIM>(sm, dot, s_attn, s_x, s_y, s_z);
  out[0] = group_sum(s_attn, lg);
  s_x = group_sum(s_x, lg);
  s_y = group_sum(s_y, lg);
  out[1] = sm.ax.pass ? (a * s_x) * (float)lv.W : 0.0f;
  out[2] = sm.ay.pass ? (a * s_y) * (float)lv.H : 0.0f;
  if constexpr (DIM == 3) {
    s_z = group_sum(s_z, lg);
    out[3] = sm.az.pass ? (a * s_z) * (float)lv.D : 0.0f;
  }
}

// Axes, corner-row offsets and anchor bin of one sample from its DIM coordinates.
template <int DIM>
__device__ inline bool sample_rows(const BwdPlan& pl, const BwdLevel& lv, bool mul24,
                                   const float* xyz, uint32_t vbase, uint32_t rs, uint32_t hsub,
                                   Sample<DIM>& sm, uint32_t (&off)[1 << DIM], uint32_t* bin) {
  bool px, py, pz = true;
  const float ux = grid_to_u(xyz[0], (float)lv.W, pl.clamp, pl.lo_g, pl.hi_g, &px);
  const float uy = grid_to_u(xyz[1], (float)lv.H, pl.clamp, pl.lo_g, pl.hi_g, &py);
  sm.ax = axis_from_u(ux, lv.W, px);
  sm.ay = axis_from_u(uy, lv.H, py);
  int tz = 0;
  bool any = (sm.ax.v0 || sm.ax.v1) && (sm.ay.v0 || sm.ay.v1);
  if constexpr (DIM == 3) {
    const float uz = grid_to_u(xyz[2], (float)lv.D, pl.clamp, pl.lo_g, pl.hi_g, &pz);
    sm.az = axis_from_u(uz, lv.D, pz);
    any = any && (sm.az.v0 || sm.az.v1);
    tz = any ? anchor_tile(sm.az, pl.tz_log2) : 0;
  }
  // byte offset of the lowest corner; 24-bit multiplies when the plan allows them
  int32_t o0;
  if (mul24) {
    o0 = __mul24(sm.ay.i0, lv.sy) + __mul24(sm.ax.i0, (int32_t)rs);
    if constexpr (DIM == 3) o0 += __mul24(sm.az.i0, lv.sz);
  } else {
    o0 = sm.ay.i0 * lv.sy + sm.ax.i0 * (int32_t)rs;
    if constexpr (DIM == 3) o0 += sm.az.i0 * lv.sz;
  }
  const uint32_t off0 = vbase + lv.base + (uint32_t)o0;
#pragma unroll
  for (int c = 0; c < (1 << DIM); ++c) {
    const uint32_t dr = ((c & 1) ? rs : 0u) + ((c & 2) ? (uint32_t)lv.sy : 0u) +
                        ((DIM == 3 && (c & 4)) ? (uint32_t)lv.sz : 0u);
    off[c] = corner_valid<DIM>(c, sm) ? off0 + dr : kOobOffset;
  }
  if (any) {
    const int tib = lv.tile_off + (tz * lv.nty + anchor_tile(sm.ay, pl.ty_log2)) * lv.ntx +
                    anchor_tile(sm.ax, pl.tx_log2);
    *bin = ((uint32_t)tib << pl.hg_log2) | hsub;
  }
  return any;
}

// One lane group of 2^lpu_log2 lanes per unit (b, q, h), with the forward's work layout:
// lane j holds channels [j*VEC, (j+1)*VEC) of the unit's grad_out row; corners outside
// the level read as zero through the buffer range check, so samples without a valid
// corner get zero gradients. PT > 0: P is a compile-time constant; each batch's
// coordinates and weights are one block load per lane, queued behind the previous
// batch's corner rows, and all SB*2^DIM corner rows of a batch are in flight together.
// LG >= 0: lanes per unit (2^LG) is a compile-time constant, else pl.lpu_log2.
// AT (plans whose levels exceed the LDS binning; PT == 0 only): instead of counting its
// samples per tile, each lane adds attn * w_c * grad_out of its channels to every valid
// corner row of the fp32 (Bc, K, H, C) sums in bf.scratch with global fp32 atomics.
// The geometry: with host shapes (pl.geom_arg) the kernel argument hg, which workgroup 0
// also stores in the workspace for the kernels after this one; else the workspace copy
// bwd_geom_kernel wrote.
template <int DIM, typename EV, typename EC, int VEC, int PT, int LG, bool AT = false>
__global__ __launch_bounds__(kGradThreads) void bwd_grad_kernel(const BwdPlan pl, const BwdBuffers bf,
                                                                const BwdGeom hg) {
  static_assert(!AT || PT == 0, "the atomic scatter is built on the generic sample loop");
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  constexpr int SB = PT > 0 ? (DIM == 2 ? (PT < 4 ? PT : 4) : (PT < 2 ? PT : 2)) : (DIM == 2 ? 2 : 1);
  typedef typename EC::T TC;
  typedef typename EV::T TV;
  extern __shared__ uint32_t s_hist[];  // [bins]
  const GeoP geo = pl.geom_arg ? (GeoP)&hg : geo_of(bf);
  if (pl.geom_arg && blockIdx.x == 0) {
    BwdGeom* dst = const_cast<BwdGeom*>(bf.geom);
    for (uint32_t i = threadIdx.x; i < sizeof(BwdGeom) / 4; i += kGradThreads)
      reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(&hg)[i];
  }
  // launches planned without the shapes run both variants; the geometry selects one
  if (AT ? (!geo->atomic || geo->invalid) : geo->atomic) return;
  const int bins = geo->bins;
  const bool mul24 = geo->mul24 != 0;
  // workgroups of one (batch, head-group) are contiguous and dealt to one XCD
  const uint32_t lb = xcd_logical_block(blockIdx.x, gridDim.x, pl.xcds);
  const uint32_t g = lb / (uint32_t)pl.wgpg;
  const uint32_t w = lb - g * (uint32_t)pl.wgpg;
  if constexpr (!AT) {
    for (int i = threadIdx.x; i < bins; i += kGradThreads) s_hist[i] = 0;
    __syncthreads();
  }

  const int lg = LG >= 0 ? LG : pl.lpu_log2;
  const uint32_t lanes = 1u << lg;
  const uint32_t lane = threadIdx.x & (lanes - 1u);
  const bool act = (int)lane < pl.nvec;
  const uint32_t gpw = (uint32_t)kGradThreads >> lg;  // unit groups per workgroup
  const uint32_t units = min((uint32_t)pl.upw, (pl.Q << pl.hg_log2) - w * (uint32_t)pl.upw);
  const int LP = pl.L * pl.P;
  const bool hm = pl.head_major != 0;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(bf.value, pl.value_bytes);
  // bytes between rows of K: one head's rows are contiguous in the head-major layout
  const uint32_t rs = (hm ? 1u : (uint32_t)pl.H) * (uint32_t)pl.C * EV::kBytes;
#pragma unroll 1
  for (uint32_t wi = threadIdx.x >> lg; wi < units; wi += gpw) {
    const BinUnit bu = bin_unit(pl, g, w, wi);
    RawVec<VB> gr = {};
    if (act) gr = glb_load<VB>(static_cast<const TV*>(bf.grad_out) + bu.bqh * pl.C + lane * VEC);
    const uint32_t slice = hm ? (bu.b * (uint32_t)pl.H + bu.h) * (uint32_t)pl.K * (uint32_t)pl.C
                              : (bu.b * (uint32_t)pl.K * (uint32_t)pl.H + bu.h) * (uint32_t)pl.C;
    const uint32_t vbase = (slice + (act ? lane : 0u) * VEC) * EV::kBytes;
    const TC* locp = static_cast<const TC*>(bf.loc) + bu.bqh * LP * DIM;
    const TC* attp = static_cast<const TC*>(bf.attn) + bu.bqh * LP;
    TC* glp = static_cast<TC*>(bf.grad_loc) + bu.bqh * LP * DIM;
    TC* gap = static_cast<TC*>(bf.grad_attn) + bu.bqh * LP;
    if constexpr (PT > 0) {
      constexpr int BPL = PT / SB;  // batches per level
      CoordBlock<EC, SB * DIM> cb;
      CoordBlock<EC, SB> ab;
      const int nbatch = pl.L * BPL;
      if (nbatch > 0) {
        load_block<EC, SB * DIM>(cb, locp);
        load_block<EC, SB>(ab, attp);
      }
      // lane j of the group keeps the gradients of batch j of every group of `lanes`
      // consecutive batches; the lanes store them together, so a wave writes whole lines
      float hga[SB], hgl[SB * DIM];
#pragma unroll
      for (int k = 0; k < SB; ++k) hga[k] = 0.0f;
#pragma unroll
      for (int k = 0; k < SB * DIM; ++k) hgl[k] = 0.0f;
#pragma unroll 1
      for (int bi = 0; bi < nbatch; ++bi) {
        const BwdLevel lv = level_at(geo, bi / BPL);
        Sample<DIM> sm[SB];
        uint32_t off[SB][NC], bin[SB];
        bool any[SB];
        float a[SB];
#pragma unroll
        for (int k = 0; k < SB; ++k) {
          float xyz[3];
#pragma unroll
          for (int d = 0; d < DIM; ++d) xyz[d] = block_elem(cb, k * DIM + d);
          bin[k] = 0;
          any[k] = sample_rows<DIM>(pl, lv, mul24, xyz, vbase, rs, bu.hsub, sm[k], off[k], &bin[k]);
          a[k] = block_elem(ab, k);
        }
        RawVec<VB> raw[SB][NC];
#pragma unroll
        for (int k = 0; k < SB; ++k)
#pragma unroll
          for (int c = 0; c < NC; ++c) raw[k][c] = buf_load<VB>(rv, off[k][c]);
        if (bi + 1 < nbatch) {
          load_block<EC, SB * DIM>(cb, locp + (bi + 1) * (SB * DIM));
          load_block<EC, SB>(ab, attp + (bi + 1) * SB);
        }
        float ga[SB], gl[SB * DIM];
#pragma unroll
        for (int k = 0; k < SB; ++k) {
          float o[DIM + 1];
          sample_grads<DIM, EV, VEC>(lv, sm[k], raw[k], gr, a[k], lg, o);
          ga[k] = o[0];
#pragma unroll
          for (int d = 0; d < DIM; ++d) gl[k * DIM + d] = o[1 + d];
          if constexpr (!AT)
            if (any[k] && lane == ((uint32_t)k & (lanes - 1u))) atomicAdd(&s_hist[bin[k]], 1u);
        }
        const uint32_t slot = (uint32_t)bi & (lanes - 1u);
        if (slot == lane) {
#pragma unroll
          for (int k = 0; k < SB; ++k) hga[k] = ga[k];
#pragma unroll
          for (int k = 0; k < SB * DIM; ++k) hgl[k] = gl[k];
        }
        if (slot == lanes - 1u || bi + 1 == nbatch) {
          // batches bi - slot .. bi: lane j stores batch bi - slot + j, all contiguous
          const int mine = bi - (int)slot + (int)lane;
          if (mine <= bi) {
            store_block<EC, SB>(gap + mine * SB, hga);
            store_block<EC, SB * DIM>(glp + mine * (SB * DIM), hgl);
          }
        }
      }
    } else {
      float gw[VEC];
      if constexpr (AT) widen<EV, VEC>(gr, gw);
      for (int l = 0; l < pl.L; ++l) {
        const BwdLevel lv = level_at(geo, l);
#pragma unroll 1
        for (int p0 = 0; p0 < pl.P; p0 += SB) {
          Sample<DIM> sm[SB];
          uint32_t off[SB][NC], bin[SB];
          bool any[SB];
          RawVec<VB> raw[SB][NC];
#pragma unroll
          for (int k = 0; k < SB; ++k) {
            const bool live = p0 + k < pl.P;
            const int s = l * pl.P + (live ? p0 + k : 0);
            float xyz[3];
#pragma unroll
            for (int d = 0; d < DIM; ++d) xyz[d] = (float)locp[s * DIM + d];
            bin[k] = 0;
            any[k] = sample_rows<DIM>(pl, lv, mul24, xyz, vbase, rs, bu.hsub, sm[k], off[k], &bin[k]);
#pragma unroll
            for (int c = 0; c < NC; ++c) raw[k][c] = buf_load<VB>(rv, live ? off[k][c] : kOobOffset);
          }
#pragma unroll
          for (int k = 0; k < SB; ++k) {
            if (p0 + k >= pl.P) continue;
            const int s = l * pl.P + p0 + k;
            float o[DIM + 1];
            const float a = (float)attp[s];
            sample_grads<DIM, EV, VEC>(lv, sm[k], raw[k], gr, a, lg, o);
            if (lane == ((uint32_t)k & (lanes - 1u))) {
              gap[s] = (TC)o[0];
#pragma unroll
              for (int d = 0; d < DIM; ++d) glp[s * DIM + d] = (TC)o[1 + d];
              if constexpr (!AT)
                if (any[k]) atomicAdd(&s_hist[bin[k]], 1u);
            }
            if constexpr (AT) {
              if (act && any[k]) {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                  if (!corner_valid<DIM>(c, sm[k])) continue;
                  const float cw = corner_weight<DIM>(c, sm[k]) * a;
                  // off is the corner row's byte offset in the value slice of this launch,
                  // channels of this lane included; the sums share its element layout
                  float* dst = bf.sums + off[k][c] / (uint32_t)EV::kBytes;
#pragma unroll
                  for (int e = 0; e < VEC; ++e) atomicAdd(dst + e, cw * gw[e]);
                }
              }
            }
          }
        }
      }
    }
  }
  if constexpr (!AT) {
    __syncthreads();
    for (int i = threadIdx.x; i < bins; i += kGradThreads)
      bf.counts[((size_t)g * bins + i) * pl.wgpg + w] = s_hist[i];
  }
}

// Binned plans, step 1: count the samples of each (tile, workgroup) from their coordinates
// alone. Same workgroup -> units mapping as the fill kernel; each workgroup histograms its
// samples per tile in LDS (integer atomics) and writes the histogram as one column of the
// tile-major count matrix. A sample with no corner inside its level gets its zero
// grad_loc and grad_attn here; every other sample's are written by the tile kernel. The
// geometry: with host shapes (pl.geom_arg) the kernel argument hg, which workgroup 0 also
// stores in the workspace for the kernels after this one; else the copy bwd_geom_kernel
// wrote. PT > 0: P is a compile-time constant and each (unit, level) block of coordinates is
// one vector load (consecutive threads read consecutive blocks); else one scalar load per
// coordinate.
template <int DIM, typename EC, int PT>
__global__ __launch_bounds__(kBlock) void bwd_count_kernel(const BwdPlan pl, const BwdBuffers bf,
                                                           const BwdGeom hg) {
  typedef typename EC::T TC;
  extern __shared__ uint32_t s_hist[];  // [bins]
  const GeoP geo = pl.geom_arg ? (GeoP)&hg : geo_of(bf);
  if (pl.geom_arg && blockIdx.x == 0) {
    BwdGeom* dst = const_cast<BwdGeom*>(bf.geom);
    for (uint32_t i = threadIdx.x; i < sizeof(BwdGeom) / 4; i += kBlock)
      reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(&hg)[i];
  }
  if (geo->atomic) return;
  const int bins = geo->bins;
  const uint32_t lb = xcd_logical_block(blockIdx.x, gridDim.x, pl.xcds);
  const uint32_t g = lb / (uint32_t)pl.wgpg;
  const uint32_t w = lb - g * (uint32_t)pl.wgpg;
  for (int i = threadIdx.x; i < bins; i += kBlock) s_hist[i] = 0;
  __syncthreads();
  const uint32_t units = min((uint32_t)pl.upw, (pl.Q << pl.hg_log2) - w * (uint32_t)pl.upw);
  const int LP = pl.L * pl.P;
  // sample si of the launch at location xyz on level lv, head hsub of the group
  auto count = [&](const BwdLevel& lv, const float* xyz, uint32_t hsub, size_t si) {
    float u[3];
    uint32_t flags;
    int tib;
    if (sample_tile<DIM>(pl, lv, xyz, u, &flags, &tib)) {
      atomicAdd(&s_hist[((uint32_t)tib << pl.hg_log2) | hsub], 1u);
    } else {
      static_cast<TC*>(bf.grad_attn)[si] = (TC)0.0f;
#pragma unroll
      for (int d = 0; d < DIM; ++d) static_cast<TC*>(bf.grad_loc)[si * DIM + d] = (TC)0.0f;
    }
  };
  constexpr int NB = 4;  // blocks (or samples) per thread in flight
  if constexpr (PT > 0) {
    const uint32_t nblk = units * (uint32_t)pl.L;
    for (uint32_t b0 = 0; b0 < nblk; b0 += NB * kBlock) {
      CoordBlock<EC, PT * DIM> cb[NB];
      size_t s0[NB];
      uint32_t hs[NB];
      int bl[NB];
      bool bv[NB];
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const uint32_t j = b0 + (uint32_t)(k * kBlock) + threadIdx.x;
        bv[k] = j < nblk;
        const uint32_t s = (bv[k] ? j : 0u) * (uint32_t)PT;
        const uint32_t wi = fdiv(s, pl.div_lp);
        bl[k] = (int)((s - wi * (uint32_t)LP) / (uint32_t)PT);
        const BinUnit bu = bin_unit(pl, g, w, wi);
        s0[k] = bu.bqh * LP + (size_t)bl[k] * PT;
        hs[k] = bu.hsub;
        if (bv[k]) load_block<EC, PT * DIM>(cb[k], static_cast<const TC*>(bf.loc) + s0[k] * DIM);
      }
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        if (!bv[k]) continue;
        const BwdLevel lv = level_at(geo, bl[k]);
#pragma unroll
        for (int p = 0; p < PT; ++p) {
          float xyz[DIM];
#pragma unroll
          for (int d = 0; d < DIM; ++d) xyz[d] = block_elem(cb[k], p * DIM + d);
          count(lv, xyz, hs[k], s0[k] + p);
        }
      }
    }
  } else {
    const uint32_t n = units * (uint32_t)LP;
    for (uint32_t r0 = 0; r0 < n; r0 += NB * kBlock) {
      float xyz[NB][DIM];
      size_t si[NB];
      uint32_t hs[NB];
      int sl[NB];
      bool sv[NB];
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const uint32_t j = r0 + (uint32_t)(k * kBlock) + threadIdx.x;
        sv[k] = j < n;
        const uint32_t s = sv[k] ? j : 0u;
        const uint32_t wi = fdiv(s, pl.div_lp);
        const uint32_t r = s - wi * (uint32_t)LP;
        sl[k] = (int)fdiv(r, pl.div_p);
        const BinUnit bu = bin_unit(pl, g, w, wi);
        si[k] = bu.bqh * LP + r;
        hs[k] = bu.hsub;
        const TC* lp = static_cast<const TC*>(bf.loc) + si[k] * DIM;
#pragma unroll
        for (int d = 0; d < DIM; ++d) xyz[k][d] = sv[k] ? (float)lp[d] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (sv[k]) count(level_at(geo, sl[k]), xyz[k], hs[k], si[k]);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < bins; i += kBlock)
    bf.counts[((size_t)g * bins + i) * pl.wgpg + w] = s_hist[i];
}

// Atomic path: clear the n fp32 sums (16-byte aligned) before the scatter.
__global__ __launch_bounds__(kBlock) void bwd_clear_sums_kernel(const BwdPlan pl, const BwdBuffers bf,
                                                                uint32_t n) {
  if (!pl.static_atomic) {  // the geometry exists already only on the device-shapes path
    const GeoP geo = geo_of(bf);
    if (!geo->atomic || geo->invalid) return;
  }
  const uint32_t stride = gridDim.x * (uint32_t)kBlock * 4u;
  for (uint32_t i = (blockIdx.x * (uint32_t)kBlock + threadIdx.x) * 4u; i < n; i += stride) {
    if (i + 4u <= n) {
      *reinterpret_cast<float4*>(bf.sums + i) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
      for (uint32_t k = i; k < n; ++k) bf.sums[k] = 0.0f;
    }
  }
}

// Atomic path: round the fp32 sums to the value dtype, VEC elements per thread and step
// (n is a multiple of VEC: C is). Invalid device shapes: every gradient becomes NaN
// (n_loc grad_loc elements and n_attn = n_loc / DIM grad_attn elements in the coord dtype).
// The sums follow the layout of value: (Bc, H, K, C) when value is head-major, whose element
// (b, k, h, c) of grad_value is read across that transpose.
template <typename EV, typename EC, int VEC>
__global__ __launch_bounds__(kBlock) void bwd_round_kernel(const BwdPlan pl, const BwdBuffers bf,
                                                           uint32_t n, uint64_t n_loc, int dim) {
  const GeoP geo = geo_of(bf);
  if (!geo->atomic) return;
  const bool nan = geo->invalid != 0;
  const uint32_t stride = gridDim.x * (uint32_t)kBlock * VEC;
  typename EV::T* dst = static_cast<typename EV::T*>(bf.grad_value);
  const uint32_t C = (uint32_t)pl.C, H = (uint32_t)pl.H, K = (uint32_t)pl.K;
  for (uint32_t i = (blockIdx.x * (uint32_t)kBlock + threadIdx.x) * VEC; i < n; i += stride) {
    uint32_t src = i;
    if (pl.head_major) {
      const uint32_t row = i / C, c = i - row * C;  // row = (b * K + k) * H + h
      const uint32_t bk = row / H, h = row - bk * H;
      const uint32_t b = bk / K, k = bk - b * K;
      src = ((b * H + h) * K + k) * C + c;
    }
    float v[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = nan ? __builtin_nanf("") : bf.sums[src + e];
    store_vec<EV, VEC>(dst + i, v);
  }
  if (nan) {
    typename EC::T* gl = static_cast<typename EC::T*>(bf.grad_loc);
    typename EC::T* ga = static_cast<typename EC::T*>(bf.grad_attn);
    const uint64_t st = (uint64_t)gridDim.x * kBlock;
    const uint64_t n_attn = n_loc / (uint64_t)dim;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n_loc; i += st) {
      gl[i] = narrow<EC>(__builtin_nanf(""));
      if (i < n_attn) ga[i] = narrow<EC>(__builtin_nanf(""));
    }
  }
}

// ------------------------------------------------------------------ 2: column scan
// One wave per tile: the tile's counts over the bin workgroups of its group become
// offsets within the tile, and its total goes to tile_n[t].
__global__ __launch_bounds__(kBlock) void bwd_colscan_kernel(const BwdPlan pl, const BwdBuffers bf) {
  const GeoP geo = geo_of(bf);
  const uint32_t t = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x & (kWave - 1);
  if (geo->atomic || t >= geo->T) return;  // the whole wave exits
  uint32_t* c = bf.counts + (size_t)t * pl.wgpg;
  uint32_t run = 0;
  // four 64-count blocks per step: their loads are issued before the first scan
  constexpr int U = 4;
  for (int base = 0; base < pl.wgpg; base += U * kWave) {
    uint32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * kWave + (int)lane;
      v[u] = i < pl.wgpg ? c[i] : 0u;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * kWave + (int)lane;
      const uint32_t inc = wave_incl_scan(v[u]);
      if (i < pl.wgpg) c[i] = run + inc - v[u];
      run += (uint32_t)__builtin_amdgcn_readlane((int)inc, kWave - 1);
    }
  }
  if (lane == 0) bf.tile_n[t] = run;
}

// ------------------------------------------------------------------ 3: plan
// One workgroup per (batch, head-group): the record totals of the group's tiles become
// first-record offsets, each tile is cut into max(1, ceil(n / R)) chunks (an empty tile
// still gets one chunk, which writes its zeros), and each chunk gets its descriptor
// {tile, first record, end record, chunks of the tile}, so a tile workgroup starts from one
// load instead of three dependent ones.
// Each workgroup first sums the totals of the tiles of all earlier groups (coalesced loads
// and a workgroup reduction), then scans its own tiles, each thread a contiguous range.
// (One workgroup for all tiles spent 14 us of C5's backward on the stores of one CU.)
__global__ __launch_bounds__(kPlanThreads) void bwd_plan_kernel(const BwdPlan pl, const BwdBuffers bf) {
  __shared__ uint32_t s_w[kPlanThreads / kWave];
  const GeoP geo = geo_of(bf);
  if (geo->atomic) return;
  const uint32_t T = geo->T, bins = (uint32_t)geo->bins;
  const uint32_t ta = blockIdx.x * bins, tb = ta + bins;
  auto chunks = [&](uint32_t n) { return max(1u, (n + pl.R - 1) / pl.R); };
  uint32_t bn = 0, bc = 0;  // records and chunks of the earlier groups
  {
    uint32_t sn = 0, sc = 0;
#pragma unroll 8
    for (uint32_t t = threadIdx.x; t < ta; t += kPlanThreads) {
      const uint32_t n = bf.tile_n[t];
      sn += n;
      sc += chunks(n);
    }
    block_excl_scan<kPlanThreads>(sn, s_w, &bn);
    block_excl_scan<kPlanThreads>(sc, s_w, &bc);
  }
  const uint32_t per = (bins + kPlanThreads - 1) / kPlanThreads;
  const uint32_t t0 = min(tb, ta + threadIdx.x * per), t1 = min(tb, t0 + per);
  // up to PB tiles per thread: their totals are loaded together and kept in registers
  constexpr uint32_t PB = 16;
  uint32_t nv[PB];
  uint32_t sn = 0, sc = 0;
  if (per <= PB) {
#pragma unroll
    for (uint32_t k = 0; k < PB; ++k) nv[k] = t0 + k < t1 ? bf.tile_n[t0 + k] : 0u;
#pragma unroll
    for (uint32_t k = 0; k < PB; ++k) {
      sn += nv[k];
      if (t0 + k < t1) sc += chunks(nv[k]);
    }
  } else {
    for (uint32_t t = t0; t < t1; ++t) {
      const uint32_t n = bf.tile_n[t];
      sn += n;
      sc += chunks(n);
    }
  }
  uint32_t tot_n, tot_c;
  uint32_t pn = bn + block_excl_scan<kPlanThreads>(sn, s_w, &tot_n);
  uint32_t pc = bc + block_excl_scan<kPlanThreads>(sc, s_w, &tot_c);
  auto place = [&](uint32_t t, uint32_t n) {
    const uint32_t nch = chunks(n);
    bf.bin_start[t] = pn;
    bf.chunk_off[t] = pc;
    for (uint32_t k = 0; k < nch; ++k)
      bf.chunks[pc + k] = make_uint4(t, pn + k * pl.R, min(pn + n, pn + (k + 1) * pl.R), nch);
    pn += n;
    pc += nch;
  };
  if (per <= PB) {
#pragma unroll
    for (uint32_t k = 0; k < PB; ++k)
      if (t0 + k < t1) place(t0 + k, nv[k]);
  } else {
    for (uint32_t t = t0; t < t1; ++t) place(t, bf.tile_n[t]);
  }
  if (tb == T && threadIdx.x == 0) {
    bf.bin_start[T] = bn + tot_n;
    bf.chunk_off[T] = bc + tot_c;
  }
}

// ------------------------------------------------------------------ records
// Words per backward record. fp32 coordinates: id | clamp flags, the pixel coordinates
// u_x, u_y[, u_z] and the weight, as fp32 (DIM + 2 words). 16-bit coordinates: id | clamp
// flags, then the sample's raw 16-bit location components and weight packed two to a word
// (x | y, then z | attn in 3D or attn in 2D: 3 words). The 16-bit values round-trip through
// fp32 exactly, and the tile kernel recomputes the pixel coordinates from them with the
// fill's grid_to_u, so it selects the same corners with the same weights. (12-byte records
// in place of 16 / 20: the fill writes and the tile kernel reads 25% / 40% fewer bytes.)
template <int DIM, typename EC>
constexpr int rec_words() {
  return record_words(DIM, EC::kBytes);
}

template <typename E>
__device__ inline float half_lo(uint32_t u) {
  if constexpr (__is_same(E, BF16)) return bf16lo(u);
  else return f16lo(u);
}

template <typename E>
__device__ inline float half_hi(uint32_t u) {
  if constexpr (__is_same(E, BF16)) return bf16hi(u);
  else return f16hi(u);
}

// ------------------------------------------------------------------ 4: fill
// Same workgroup -> units mapping as the count kernel. In rounds of at most
// kFillStage samples (PT > 0: the workgroup's samples in memory order over all levels;
// otherwise level by level): rank each sample within its bin (LDS atomics), scan the
// round's per-bin counts, place the records in LDS sorted by bin, and copy them out so that
// consecutive threads write consecutive records of one bin.
template <int DIM, typename EC, int PT>
__global__ __launch_bounds__(kBlock) void bwd_fill_kernel(const BwdPlan pl, const BwdBuffers bf) {
  typedef typename EC::T TC;
  constexpr int RW = rec_words<DIM, EC>();
  constexpr int KP = kFillStage / kBlock;  // samples per thread per round
  extern __shared__ __attribute__((aligned(16))) uint32_t s_fill[];
  const GeoP geo = geo_of(bf);
  if (geo->atomic) return;
  const int bins = geo->bins;
  uint32_t* s_rec = s_fill;                // [kFillStage * RW] records sorted by bin (16-byte aligned)
  uint32_t* s_dst = s_rec + kFillStage * RW;  // [kFillStage] global record index of each
  uint32_t* s_base = s_dst + kFillStage;   // [bins] next global record of each bin
  uint32_t* s_cnt = s_base + bins;         // [bins] round counts -> round offsets
  uint32_t* s_w = s_cnt + bins;            // [kBlock / kWave]
  // 2D: a group's workgroups in a contiguous range per XCD, so its record lines are
  // written through one L2 (C2 fill 48 -> 44 us); 3D keeps them dealt round-robin
  // (C5 105 against 110 us grouped)
  const uint32_t lbk = DIM == 2 ? xcd_logical_block(blockIdx.x, gridDim.x, pl.xcds) : blockIdx.x;
  const uint32_t g = lbk / (uint32_t)pl.wgpg;
  const uint32_t w = lbk - g * (uint32_t)pl.wgpg;
  for (int i = threadIdx.x; i < bins; i += kBlock)
    s_base[i] = bf.bin_start[(size_t)g * bins + i] + bf.counts[((size_t)g * bins + i) * pl.wgpg + w];
  const uint32_t units = min((uint32_t)pl.upw, (pl.Q << pl.hg_log2) - w * (uint32_t)pl.upw);
  const int LP = pl.L * pl.P;
  // After a round's ranking: scan the round's counts of bins [b0, b1), place the records in
  // LDS sorted by bin, copy them out (consecutive threads write consecutive records of a
  // bin) and advance the bins' global positions. key = bin << 16 | rank, or ~0u.
  auto finish_round = [&](const uint32_t (&key)[KP], const uint32_t (&rw)[KP][RW], uint32_t b0,
                          uint32_t b1) {
    lds_sync();
    // exclusive scan of the round's bin counts: each thread sums a run of consecutive bins,
    // one block scan of those sums, then each thread writes its run's offsets (one block
    // scan, two barriers, however many bins; a block scan per 256 bins took ten barriers
    // per round at C5's 1170 bins)
    uint32_t carry;
    {
      const uint32_t per = (b1 - b0 + kBlock - 1) / kBlock;
      const uint32_t j0 = min(b1, b0 + threadIdx.x * per), j1 = min(b1, j0 + per);
      uint32_t sum = 0;
      for (uint32_t j = j0; j < j1; ++j) sum += s_cnt[j];
      uint32_t run = block_excl_scan<kBlock>(sum, s_w, &carry);
      for (uint32_t j = j0; j < j1; ++j) {
        const uint32_t v = s_cnt[j];
        s_cnt[j] = run;
        run += v;
      }
    }
    lds_sync();
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      if (key[k] == 0xffffffffu) continue;
      const uint32_t bin = key[k] >> 16, rank = key[k] & 0xffffu, pos = s_cnt[bin] + rank;
      uint32_t* rec = s_rec + pos * RW;
      if constexpr (RW == 4) {
        *reinterpret_cast<uint4*>(rec) = make_uint4(rw[k][0], rw[k][1], rw[k][2], rw[k][3]);
      } else {
#pragma unroll
        for (int i = 0; i < RW; ++i) rec[i] = rw[k][i];
      }
      s_dst[pos] = s_base[bin] + rank;
    }
    lds_sync();
    if constexpr (RW == 4) {
      // 16-byte records: one LDS read and one 16-byte store per record
      for (uint32_t r = threadIdx.x; r < carry; r += kBlock) {
        const uint4 v = reinterpret_cast<const uint4*>(s_rec)[r];
        reinterpret_cast<uint4*>(bf.records)[s_dst[r]] = v;
      }
    } else {
      // one record per thread: its destination is read once
      for (uint32_t r = threadIdx.x; r < carry; r += kBlock) {
        uint32_t v[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) v[i] = s_rec[r * RW + i];
        uint32_t* d = bf.records + (size_t)s_dst[r] * RW;
#pragma unroll
        for (int i = 0; i < RW; ++i) d[i] = v[i];
      }
    }
    lds_sync();
    for (uint32_t i = b0 + threadIdx.x; i < b1; i += kBlock)
      s_base[i] += (i + 1 < b1 ? s_cnt[i + 1] : carry) - s_cnt[i];
    lds_sync();  // the next round clears s_cnt
  };
  // rank sample k of a round from its inputs; its record stays in registers
  auto rank = [&](int k, const BwdLevel& lv, const float* xyz, float at, uint32_t qp, uint32_t hsub,
                  uint32_t (&key)[KP], uint32_t (&rw)[KP][RW]) {
    float u[3];
    uint32_t flags;
    int tib;
    if (!sample_tile<DIM>(pl, lv, xyz, u, &flags, &tib)) return;
    const uint32_t bin = ((uint32_t)tib << pl.hg_log2) | hsub;
    key[k] = (bin << 16) | atomicAdd(&s_cnt[bin], 1u);
    rw[k][0] = qp | flags;
    if constexpr (RW == 3) {
      // the raw 16-bit inputs (xyz and at hold them exactly)
      rw[k][1] = pack2<EC>(xyz[0], xyz[1]);
      rw[k][2] = DIM == 3 ? pack2<EC>(xyz[DIM - 1], at) : pack2<EC>(at, 0.0f);
    } else {
      rw[k][1] = as_u32(u[0]);
      rw[k][2] = as_u32(u[1]);
      if constexpr (DIM == 3) rw[k][3] = as_u32(u[2]);
      rw[k][RW - 1] = as_u32(at);
    }
  };
  if constexpr (PT > 0) {
    // All of the workgroup's samples in memory order (unit, level, point), in rounds over
    // every bin of the group: thread t takes samples [t * KP, t * KP + KP) of a round, i.e.
    // KP / PT whole (unit, level) blocks, each one vector load of its PT coordinates and one
    // of its weights; consecutive threads read consecutive blocks. (Rounds per level, with
    // one scalar load per coordinate and a 64-byte stride between threads, left the fill
    // bound by the load pipeline: C2 fill 42 -> 34 us, C5 103 -> 91 us.)
    constexpr int NBK = KP / (PT > 0 ? PT : 1);
    static_assert(KP % (PT > 0 ? PT : 1) == 0, "a thread takes whole (unit, level) blocks");
    const uint32_t n = units * (uint32_t)LP;
    for (uint32_t r0 = 0; r0 < n; r0 += kFillStage) {
      const uint32_t nr = min((uint32_t)kFillStage, n - r0);  // a multiple of PT
      for (int i = threadIdx.x; i < bins; i += kBlock) s_cnt[i] = 0;
      lds_sync();
      CoordBlock<EC, PT * DIM> cb[NBK];
      CoordBlock<EC, PT> ab[NBK];
      uint32_t bq[NBK], bh[NBK];
      int bl[NBK];
      bool bv[NBK];
#pragma unroll
      for (int bk = 0; bk < NBK; ++bk) {
        const uint32_t j = threadIdx.x * (uint32_t)KP + (uint32_t)(bk * PT);
        bv[bk] = j < nr;
        const uint32_t s = r0 + (bv[bk] ? j : 0u);
        const uint32_t wi = fdiv(s, pl.div_lp);
        const int l = (int)((s - wi * (uint32_t)LP) / (uint32_t)PT);
        const BinUnit bu = bin_unit(pl, g, w, wi);
        const size_t s0 = bu.bqh * LP + (size_t)l * PT;
        load_block<EC, PT * DIM>(cb[bk], static_cast<const TC*>(bf.loc) + s0 * DIM);
        load_block<EC, PT>(ab[bk], static_cast<const TC*>(bf.attn) + s0);
        bq[bk] = bu.q;
        bh[bk] = bu.hsub;
        bl[bk] = l;
      }
      uint32_t key[KP];
      uint32_t rw[KP][RW];
#pragma unroll
      for (int k = 0; k < KP; ++k) key[k] = 0xffffffffu;
#pragma unroll
      for (int bk = 0; bk < NBK; ++bk) {
        if (!bv[bk]) continue;
        const BwdLevel lv = level_at(geo, bl[bk]);
#pragma unroll
        for (int p = 0; p < PT; ++p) {
          float xyz[DIM];
#pragma unroll
          for (int d = 0; d < DIM; ++d) xyz[d] = block_elem(cb[bk], p * DIM + d);
          rank(bk * PT + p, lv, xyz, block_elem(ab[bk], p), bq[bk] * (uint32_t)PT + (uint32_t)p,
               bh[bk], key, rw);
        }
      }
      finish_round(key, rw, 0u, (uint32_t)bins);
    }
  } else {
    for (int l = 0; l < pl.L; ++l) {
      const BwdLevel lv = level_at(geo, l);
      const uint32_t lb0 = (uint32_t)lv.tile_off << pl.hg_log2;
      const uint32_t lb1 = (uint32_t)(lv.tile_off + lv.ntiles) << pl.hg_log2;
      const uint32_t n = units * (uint32_t)pl.P;
      for (uint32_t r0 = 0; r0 < n; r0 += kFillStage) {
        const uint32_t nr = min((uint32_t)kFillStage, n - r0);
        for (uint32_t i = lb0 + threadIdx.x; i < lb1; i += kBlock) s_cnt[i] = 0;
        lds_sync();
        // every coordinate and weight load of the round first (no branch between them, so
        // they are in flight together), then rank each sample within its bin. (Prefetching
        // the next round's loads across the round's barriers was slower.)
        float xyz[KP][DIM], at[KP];
        uint32_t qp[KP], hs[KP];
#pragma unroll
        for (int k = 0; k < KP; ++k) {
          const uint32_t j = threadIdx.x + k * kBlock;
          const uint32_t js = r0 + (j < nr ? j : 0u);
          const uint32_t wi = fdiv(js, pl.div_p), p = js - wi * (uint32_t)pl.P;
          const BinUnit bu = bin_unit(pl, g, w, wi);
          const size_t si = bu.bqh * LP + (size_t)l * pl.P + p;
          const TC* lp = static_cast<const TC*>(bf.loc) + si * DIM;
#pragma unroll
          for (int d = 0; d < DIM; ++d) xyz[k][d] = (float)lp[d];
          at[k] = (float)static_cast<const TC*>(bf.attn)[si];
          qp[k] = bu.q * (uint32_t)pl.P + p;
          hs[k] = bu.hsub;
        }
        uint32_t key[KP];
        uint32_t rw[KP][RW];
#pragma unroll
        for (int k = 0; k < KP; ++k) {
          key[k] = 0xffffffffu;
          if (threadIdx.x + k * kBlock < nr) rank(k, lv, xyz[k], at[k], qp[k], hs[k], key, rw);
        }
        finish_round(key, rw, lb0, lb1);
      }
    }
  }
}

// Axes of a staged record (16-bit records: the fill's grid_to_u on the same inputs).
template <int DIM, typename EC>
__device__ inline Sample<DIM> record_sample(const uint32_t* rec, const BwdLevel& lv, const BwdPlan& pl) {
  Sample<DIM> sm;
  if constexpr (rec_words<DIM, EC>() == 3) {
    bool px, py, pz = true;
    const float ux = grid_to_u(half_lo<EC>(rec[1]), (float)lv.W, pl.clamp, pl.lo_g, pl.hi_g, &px);
    const float uy = grid_to_u(half_hi<EC>(rec[1]), (float)lv.H, pl.clamp, pl.lo_g, pl.hi_g, &py);
    sm.ax = axis_from_u(ux, lv.W, px);
    sm.ay = axis_from_u(uy, lv.H, py);
    if constexpr (DIM == 3) {
      const float uz = grid_to_u(half_lo<EC>(rec[2]), (float)lv.D, pl.clamp, pl.lo_g, pl.hi_g, &pz);
      sm.az = axis_from_u(uz, lv.D, pz);
    }
  } else {
    const uint32_t id = rec[0];
    sm.ax = axis_from_u(__builtin_bit_cast(float, rec[1]), lv.W, (id & kRecPassX) != 0);
    sm.ay = axis_from_u(__builtin_bit_cast(float, rec[2]), lv.H, (id & kRecPassY) != 0);
    if constexpr (DIM == 3) sm.az = axis_from_u(__builtin_bit_cast(float, rec[3]), lv.D, (id & kRecPassZ) != 0);
  }
  return sm;
}

// The attention weight of a staged record.
template <int DIM, typename EC>
__device__ inline float record_attn(const uint32_t* rec) {
  if constexpr (rec_words<DIM, EC>() == 3) return DIM == 3 ? half_hi<EC>(rec[2]) : half_lo<EC>(rec[2]);
  else return __builtin_bit_cast(float, rec[DIM + 1]);
}

template <int DIM>
__device__ inline int corner_cell(const Region& rg, const TileCoord& tc, const Sample<DIM>& sm, int cc) {
  return region_cell(rg, sm.ax.i0 + (cc & 1) - tc.X0, sm.ay.i0 + ((cc >> 1) & 1) - tc.Y0,
                     DIM == 3 ? sm.az.i0 + ((cc >> 2) & 1) - tc.Z0 : 0);
}

// ------------------------------------------------------------------ 5: tile kernel
// N fp32 values from LDS (one 16-byte read for N == 4).
template <int N>
__device__ inline void lds_f32(const char* p, float (&v)[N]) {
  if constexpr (N == 4) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = reinterpret_cast<const float*>(p)[i];
  }
}

// N staged elements of type E from LDS, widened to fp32 (one 8-byte read for four 16-bit
// elements, one 16-byte read for four fp32 ones).
template <typename E, int N>
__device__ inline void lds_elems(const char* p, float (&v)[N]) {
  if constexpr (E::kBytes == 4) lds_f32<N>(p, v);
  else widen<E, N>(*reinterpret_cast<const RawVec<N * 2>*>(p), v);
}

// Exclusive scan, in place, of the n + 1 counters c[0..n] of a region by one wave (c[n] is
// zero before, the total after). c is 16-byte aligned and padded to a multiple of four
// counters; each lane scans a run of whole quads (one 16-byte read and write each; a
// region of up to 255 cells is one quad per lane). Every lane of the wave must call it.
__device__ inline void wave_scan_counts(uint32_t* c, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  const int nq = (n + 4) >> 2;
  uint4* q = reinterpret_cast<uint4*>(c);
  if (nq <= kWave) {
    const uint4 v = lane < nq ? q[lane] : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t sum = v.x + v.y + v.z + v.w;
    const uint32_t run = wave_incl_scan(sum) - sum;
    if (lane < nq) q[lane] = make_uint4(run, run + v.x, run + v.x + v.y, run + v.x + v.y + v.z);
    return;
  }
  const int per = (nq + kWave - 1) / kWave;
  const int i0 = lane * per, i1 = min(nq, i0 + per);
  uint32_t sum = 0;
  for (int i = i0; i < i1; ++i) {
    const uint4 v = q[i];
    sum += v.x + v.y + v.z + v.w;
  }
  uint32_t run = wave_incl_scan(sum) - sum;
  for (int i = i0; i < i1; ++i) {
    const uint4 v = q[i];
    q[i] = make_uint4(run, run + v.x, run + v.x + v.y, run + v.x + v.y + v.z);
    run += v.x + v.y + v.z + v.w;
  }
}

// One workgroup (kTileThreads<DIM> threads) per chunk of a tile's records, in sub-batches of
// S <= kTileThreads<DIM> records; thread t owns record t of the sub-batch in registers. LDS
// holds the value rows of the tile's region (staged once per chunk), the sub-batch's
// grad_out rows in the value dtype, its (attn * corner weight, row byte offset) entries
// sorted by region cell, and two sets of per-cell counters (one being filled while the
// other is cleared). Per sub-batch, four barriers:
//   1. every wave stages the grad_out rows of its 64 records (four lanes per 16-byte
//      chunk group, the row index handed over with ds_bpermute) while each record's
//      owner counts its corners per region cell (LDS integer atomics give the ranks);
//   2. one wave scans the counters; the other counter set is cleared; each owner forms
//      its record's corner dot products <grad_out, v_c> from LDS and stores the sample's
//      grad_attn and clamp-masked grad_loc;
//   3. owners place their entries at offset + rank and fetch the next sub-batch's record;
//   4. the thread owning (region cell, channel chunk) sums its cell's entries into fp32
//      registers.
template <int DIM, typename EV, typename EC, int VEC, bool DOTS>
__global__ __launch_bounds__(kTileThreads<DIM>, kTileWavesPerSimd) void bwd_tile_kernel(const BwdPlan pl,
                                                                const BwdBuffers bf) {
  constexpr int NT = kTileThreads<DIM>;
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  constexpr int RW = rec_words<DIM, EC>();  // words per record
  // channels per owner item: 16 staged bytes, so the lanes of one cell read a staged row
  // conflict-free; owner items per thread
  constexpr int OV = tile_owner_vec(VEC, EV::kBytes);
  constexpr int MI = tile_max_items(OV);
  constexpr int GB = 4;                   // grad_out chunk loads in flight per thread
  typedef typename EV::T TV;
  typedef typename EC::T TC;
  extern __shared__ __attribute__((aligned(16))) char s_mem[];

  // Chunks are dealt to XCDs in contiguous ranges (workgroup i runs on XCD i % xcds), so the
  // chunks of one (batch, head-group) share an XCD and its L2. When the groups divide evenly
  // over the XCDs, each XCD takes whole groups, whose chunks run coarsest level first: the
  // longest chunks start first. (Equal-size ranges split groups, and a group cut at the end
  // of one XCD's range left its coarse chunks to start last: C5 tile 487 -> 435 us.)
  const GeoP geo = geo_of(bf);
  if (geo->atomic) return;
  const uint32_t xcds = pl.xcds;
  const uint32_t slot = blockIdx.x / xcds, x = blockIdx.x % xcds;
  uint32_t c;
  if ((uint32_t)pl.groups % xcds == 0u) {
    const uint32_t tiles_x = (uint32_t)pl.groups / xcds * (uint32_t)geo->bins;
    const uint32_t c0 = bf.chunk_off[x * tiles_x], c1 = bf.chunk_off[(x + 1) * tiles_x];
    c = c0 + slot;
    if (c >= c1) return;  // the whole workgroup exits
  } else {
    const uint32_t total = bf.chunk_off[geo->T];
    const uint32_t per = (total + xcds - 1) / xcds;
    if (slot >= per) return;
    c = x * per + slot;
    if (c >= total) return;
  }
  const uint4 cd = bf.chunks[c];
  const uint32_t t = cd.x, beg = cd.y, end = cd.z, nch = cd.w;
  BwdLevel lv;
  const TileCoord tc = decode_tile(pl, geo, t, &lv);

  const uint32_t S = pl.S;
  const uint32_t grow = pl.grow;  // bytes between staged grad_out rows (value dtype)
  // bytes between staged value rows: an odd number of 16-byte slots, so the same chunk of
  // random rows falls in every slot of a bank row, not in every second or fourth one
  const uint32_t vrow = pl.vrow;
  char* s_g = s_mem;                                                   // [S][grow] grad_out
  uint2* s_ent = reinterpret_cast<uint2*>(s_g + pl.lds_g_bytes);       // [S * NC]
  // two counter sets of rcells + 1 counters, each padded to whole quads (16-byte aligned:
  // S * grow and S * NC * 8 are multiples of 16)
  uint32_t* s_cnt2 = reinterpret_cast<uint32_t*>(s_ent + (size_t)S * NC);
  const int ncp = (pl.rcells + 4) & ~3;  // counter-set stride, sized for a full region
  char* s_v = reinterpret_cast<char*>(s_cnt2 + 2 * ncp);  // [region cells][vrow] value rows
  // compact region: the owner items and counters cover only its cells (a partial tile on a
  // coarse level's edge spreads its entries over all owner threads instead of the few whose
  // fixed-layout cells it touches: C2 level-3 edge chunks 176 -> 110 us, tile kernel 174 -> 161 us)
  const Region rg = tile_region(pl, tc, lv);
  const int ncell_r = rg.ex * rg.ey * rg.ez;
  const uint32_t nvec = (uint32_t)pl.nvec;
  const int tid = (int)threadIdx.x;
  const int lane = tid & (kWave - 1), wv = tid >> 6;
  const TV* gout = static_cast<const TV*>(bf.grad_out) + ((size_t)tc.b * pl.Q * pl.H + tc.h) * pl.C;
  const size_t grad_q_stride = (size_t)pl.H * pl.C;  // elements between queries of grad_out

  // the region's value rows -> LDS, once per chunk: every corner of the chunk's samples
  // (their <grad_out, v_c> dot products give grad_attn and grad_loc)
  if constexpr (DOTS) {
    // in rounds of KS items per thread, every load of a round issued before its LDS stores
    // (one storing each load before the next was issued left the chunk's prologue waiting
    // for KS memory round trips in a row)
    constexpr int KS = 4;
    const TV* val = static_cast<const TV*>(bf.value);
    const RegionSplit rs = region_split(rg);
    const int nit = ncell_r * (int)nvec;
    for (int i0 = tid; i0 < nit; i0 += KS * NT) {
      RawVec<VB> v[KS];
      uint32_t dst[KS];
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const int i = i0 + k * NT;
        dst[k] = 0xffffffffu;
        if (i < nit) {
          const int cell = (int)fdiv((uint32_t)i, pl.div_nvec), ch = i - cell * (int)nvec;
          int rx, ry, rz;
          split_cell(rs, cell, rx, ry, rz);
          const uint32_t row = (uint32_t)lv.start +
                               ((uint32_t)(tc.Z0 + rz) * lv.H + (tc.Y0 + ry)) * lv.W + (tc.X0 + rx);
          const size_t e = pl.head_major ? (((size_t)tc.b * pl.H + tc.h) * pl.K + row) * pl.C
                                         : (((size_t)tc.b * pl.K + row) * pl.H + tc.h) * pl.C;
          v[k] = glb_load<VB>(val + e + ch * VEC);
          dst[k] = (uint32_t)cell * vrow + (uint32_t)ch * VB;
        }
      }
#pragma unroll
      for (int k = 0; k < KS; ++k)
        if (dst[k] != 0xffffffffu) *reinterpret_cast<RawVec<VB>*>(s_v + dst[k]) = v[k];
    }
  }

  const int onv = pl.onv;
  float acc[MI][OV];
#pragma unroll
  for (int m = 0; m < MI; ++m)
#pragma unroll
    for (int k = 0; k < OV; ++k) acc[m][k] = 0.0f;

  for (int i = tid; i < 2 * ncp; i += NT) s_cnt2[i] = 0u;
  uint32_t rec[RW];
#pragma unroll
  for (int k = 0; k < RW; ++k) rec[k] = 0u;
  if ((uint32_t)tid < S && beg + (uint32_t)tid < end) {
#pragma unroll
    for (int k = 0; k < RW; ++k) rec[k] = bf.records[(size_t)(beg + tid) * RW + k];
  }
  lds_sync();

  int par = 0;
  for (uint32_t sb = beg; sb < end; sb += S, par ^= 1) {
    const uint32_t nrec = min(S, end - sb);
    uint32_t* s_cnt = s_cnt2 + par * ncp;
    const bool has = (uint32_t)tid < nrec;

    // 1. grad_out rows -> LDS in the value dtype; corner ranks
    const uint32_t q = has ? fdiv(rec[0] & kRecIdMask, pl.div_p) : 0u;
    Sample<DIM> sm;
    uint32_t slot[NC];  // (region cell << 16) | rank within the cell, or ~0u: no entry
    for (uint32_t m0 = 0; m0 < nvec; m0 += GB) {
      RawVec<VB> gr[GB];
      uint32_t dst[GB];
      // every load unconditional, so all of them are in flight together (loads under a
      // per-lane branch were each issued only after the previous one had returned): chunks past
      // the row's end re-load its last chunk, rows past the sub-batch's end load the row of
      // query 0 (q is 0 without a record), and neither is stored
#pragma unroll
      for (int k = 0; k < GB; ++k) {
        const uint32_t m = min(m0 + (uint32_t)k, nvec - 1u);
        const uint32_t jj = m * kWave + (uint32_t)lane;
        const uint32_t lr = fdiv(jj, pl.div_nvec), ch = jj - lr * nvec;
        const uint32_t qq = (uint32_t)__builtin_amdgcn_ds_bpermute((int)(lr << 2), (int)q);
        const uint32_t r = (uint32_t)wv * kWave + lr;
        gr[k] = glb_load<VB>(gout + (size_t)qq * grad_q_stride + ch * VEC);
        dst[k] = m0 + (uint32_t)k < nvec && r < nrec ? r * grow + ch * (uint32_t)VB : 0xffffffffu;
      }
      if (m0 == 0 && has) {
        // the owner's corners, while the first row loads are in flight
        sm = record_sample<DIM, EC>(rec, lv, pl);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          const int ce = corner_cell<DIM>(rg, tc, sm, cc);
          slot[cc] = 0xffffffffu;
          if (corner_valid<DIM>(cc, sm) && ce >= 0)
            slot[cc] = ((uint32_t)ce << 16) | atomicAdd(&s_cnt[ce], 1u);
        }
      }
#pragma unroll
      for (int k = 0; k < GB; ++k)
        if (dst[k] != 0xffffffffu) *reinterpret_cast<RawVec<VB>*>(s_g + dst[k]) = gr[k];
    }
    lds_sync();

    // 2. scan this set of counters; clear the other (last read in the previous sub-batch);
    // each owner forms its record's corner dot products from the staged grad_out row and
    // region rows and stores the sample's grad_attn and clamp-masked grad_loc
    if (wv == 0) wave_scan_counts(s_cnt, ncell_r);
    {
      uint32_t* o = s_cnt2 + (par ^ 1) * ncp;
      for (int i = tid; i <= ncell_r; i += NT) o[i] = 0u;
    }
    if (DOTS && has) {
      uint32_t vo[NC];
      float dot[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        vo[cc] = slot[cc] != 0xffffffffu ? (slot[cc] >> 16) * vrow : 0u;
        dot[cc] = 0.0f;
      }
      const char* gp = s_g + (uint32_t)tid * grow;
      for (uint32_t j = 0; j < nvec; ++j) {
        const RawVec<VB> gk = *reinterpret_cast<const RawVec<VB>*>(gp + j * VB);
        if constexpr (EV::kBytes == 2 && VEC >= 2) {
          // 16-bit grad_out and value: each pair of channels is one dot2 of the raw dwords
          // (exact products, fp32 sum)
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) {
            const RawVec<VB> r = *reinterpret_cast<const RawVec<VB>*>(s_v + vo[cc] + j * VB);
#pragma unroll
            for (int e = 0; e < VEC / 2; ++e) dot[cc] = dot2_acc<EV>(raw_dword(r, e), raw_dword(gk, e), dot[cc]);
          }
        } else {
          float g[VEC];
          widen<EV, VEC>(gk, g);
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) {
            float v[VEC];
            widen<EV, VEC>(*reinterpret_cast<const RawVec<VB>*>(s_v + vo[cc] + j * VB), v);
#pragma unroll
            for (int e = 0; e < VEC; ++e) dot[cc] = __builtin_fmaf(g[e], v[e], dot[cc]);
          }
        }
      }
      // corners outside the level or the region read zero (the zero padding)
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
        if (slot[cc] == 0xffffffffu) dot[cc] = 0.0f;
      float s_attn, s_x, s_y, s_z;
      corner_grads<DIM>(sm, dot, s_attn, s_x, s_y, s_z);
      const float a = record_attn<DIM, EC>(rec);
      const uint32_t p = (rec[0] & kRecIdMask) - q * (uint32_t)pl.P;
      const size_t si = (((size_t)tc.b * pl.Q + q) * pl.H + tc.h) * (size_t)(pl.L * pl.P) +
                        (size_t)tc.l * pl.P + p;
      TC* gl = static_cast<TC*>(bf.grad_loc) + si * DIM;
      static_cast<TC*>(bf.grad_attn)[si] = (TC)s_attn;
      float o[DIM];
      o[0] = sm.ax.pass ? (a * s_x) * (float)lv.W : 0.0f;
      o[1] = sm.ay.pass ? (a * s_y) * (float)lv.H : 0.0f;
      if constexpr (DIM == 3) o[2] = sm.az.pass ? (a * s_z) * (float)lv.D : 0.0f;
      // scattered stores cost a request each: the 2D pair as one store where aligned
      if constexpr (DIM == 2) {
        if (pl.coords_aligned) {
          store_block<EC, 2>(gl, o);
        } else {
          gl[0] = (TC)o[0];
          gl[1] = (TC)o[1];
        }
      } else if constexpr (EC::kBytes == 2) {
        // three 16-bit values: the 4-byte-aligned pair as one store
        if (pl.coords_aligned && (si & 1u) == 0u) {
          *reinterpret_cast<uint32_t*>(gl) = pack2<EC>(o[0], o[1]);
          gl[2] = (TC)o[2];
        } else if (pl.coords_aligned) {
          gl[0] = (TC)o[0];
          *reinterpret_cast<uint32_t*>(gl + 1) = pack2<EC>(o[1], o[2]);
        } else {
#pragma unroll
          for (int d = 0; d < DIM; ++d) gl[d] = (TC)o[d];
        }
      } else {
#pragma unroll
        for (int d = 0; d < DIM; ++d) gl[d] = (TC)o[d];
      }
    }
    lds_sync();

    // 3. place the entries; fetch the next sub-batch's record
    if (has) {
      const float a = record_attn<DIM, EC>(rec);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        if (slot[cc] != 0xffffffffu) {
          const float cw = corner_weight<DIM>(cc, sm) * a;
          s_ent[s_cnt[slot[cc] >> 16] + (slot[cc] & 0xffffu)] = make_uint2(as_u32(cw), (uint32_t)tid * grow);
        }
      }
    }
    {
      const uint32_t nx = sb + S + (uint32_t)tid;
      if ((uint32_t)tid < S && nx < end) {
#pragma unroll
        for (int k = 0; k < RW; ++k) rec[k] = bf.records[(size_t)nx * RW + k];
      }
    }
    lds_sync();

    // 4. owner pass: fp32 register accumulation per (region cell, channel chunk). Every
    // item's entry range is read first (one LDS round trip for all of them); within an item,
    // four entries per step (their entry and row reads are independent, so their LDS
    // latencies overlap) and a tail of up to three entries in one step (entries past the end
    // re-read the first one with weight zero). Reading the next step's entries during a step
    // was slower: the register copies cost more issue than the round trip they hide.
    uint32_t eb[MI], ee[MI];
#pragma unroll
    for (int m = 0; m < MI; ++m) {
      const int it = tid + m * NT;
      eb[m] = ee[m] = 0u;
      if (it < ncell_r * onv) {
        const int ce = (int)fdiv((uint32_t)it, pl.div_onv);
        eb[m] = s_cnt[ce];
        ee[m] = s_cnt[ce + 1];
      }
    }
#pragma unroll
    for (int m = 0; m < MI; ++m) {
      const int it = tid + m * NT;
      if (it >= ncell_r * onv) continue;
      const int ce = (int)fdiv((uint32_t)it, pl.div_onv), ch = it - ce * onv;
      const char* gb = s_g + ch * (OV * EV::kBytes);
      uint32_t e = eb[m];
      const uint32_t e1 = ee[m];
      for (; e + 4 <= e1; e += 4) {
        uint2 en[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) en[j] = s_ent[e + j];
        float gv[4][OV];
#pragma unroll
        for (int j = 0; j < 4; ++j) lds_elems<EV, OV>(gb + en[j].y, gv[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int k = 0; k < OV; ++k) acc[m][k] = __builtin_fmaf(as_float(en[j].x), gv[j][k], acc[m][k]);
      }
      if (e < e1) {
        const uint32_t r = e1 - e;  // 1 .. 3
        const uint2 t0 = s_ent[e];
        const uint2 t1 = s_ent[r > 1 ? e + 1 : e];
        const uint2 t2 = s_ent[r > 2 ? e + 2 : e];
        float g0[OV], g1[OV], g2[OV];
        lds_elems<EV, OV>(gb + t0.y, g0);
        lds_elems<EV, OV>(gb + t1.y, g1);
        lds_elems<EV, OV>(gb + t2.y, g2);
        const float w1 = r > 1 ? as_float(t1.x) : 0.0f, w2 = r > 2 ? as_float(t2.x) : 0.0f;
#pragma unroll
        for (int k = 0; k < OV; ++k) {
          acc[m][k] = __builtin_fmaf(as_float(t0.x), g0[k], acc[m][k]);
          acc[m][k] = __builtin_fmaf(w1, g1[k], acc[m][k]);
          acc[m][k] = __builtin_fmaf(w2, g2[k], acc[m][k]);
        }
      }
    }
    lds_sync();  // LDS of this sub-batch is reused by the next one
  }

  const RegionSplit rs_out = region_split(rg);
  // write the region: interior cells of a one-chunk tile directly in the value dtype;
  // edge cells, halo cells inside the level and all cells of a split tile as fp32 partials
  // for the fold kernel
#pragma unroll
  for (int m = 0; m < MI; ++m) {
    const int it = (int)threadIdx.x + m * NT;
    if (it >= ncell_r * onv) continue;
    const int cell = (int)fdiv((uint32_t)it, pl.div_onv), ch = it - cell * onv;
    int rx, ry, rz;
    split_cell(rs_out, cell, rx, ry, rz);
    const int x = tc.X0 + rx, y = tc.Y0 + ry, z = tc.Z0 + rz;
    const bool owned = rx < pl.TX && ry < pl.TY && rz < pl.TZ;
    const bool interior = owned && rx > 0 && ry > 0 && (DIM == 2 || rz > 0);
    if (nch == 1 && interior) {
      const uint32_t row = (uint32_t)lv.start + ((uint32_t)z * lv.H + y) * lv.W + x;
      store_vec<EV, OV>(static_cast<TV*>(bf.grad_value) +
                            (((size_t)tc.b * pl.K + row) * pl.H + tc.h) * pl.C + ch * OV,
                        acc[m]);
    } else {
      // partials in the fold's full-region layout
      const int full = (rz * pl.RY + ry) * pl.RX + rx;
      float* dst = bf.scratch + ((size_t)c * pl.rcells + full) * pl.C + ch * OV;
      store_vec<F32, OV>(dst, acc[m]);
    }
  }
}

// ------------------------------------------------------------------ 6: fold
// o += src[j * stride] for j = 0 .. n-1, in that order; four chunks' loads are issued
// before their additions so their latencies overlap.
template <int VEC>
__device__ inline void add_partials(float (&o)[VEC], const float* src, size_t stride, uint32_t n) {
  uint32_t j = 0;
  for (; j + 4 <= n; j += 4) {
    float v[4][VEC];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < VEC; ++k) v[u][k] = src[(j + u) * stride + k];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < VEC; ++k) o[k] += v[u][k];
  }
  for (; j < n; ++j)
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] += src[j * stride + k];
}

// One workgroup per tile. Sums, for every edge cell (and every cell of a split tile), the
// partials of the tile's own chunks and then the halo partials of the chunks of the lower
// neighbours whose halo covers the cell, and writes the cell in the value dtype. The
// neighbours' chunk ranges are the same for the whole tile and are read once. When the tile
// and its neighbours are one chunk each (the common case), a cell's partial loads are all
// issued before the first addition, in one round trip instead of one per source (C5 fold
// 88 -> 75 us, C2 15 -> 14 us); the additions keep the same order either way.
template <int DIM, typename EV, int VEC>
__global__ __launch_bounds__(kBlock) void bwd_fold_kernel(const BwdPlan pl, const BwdBuffers bf) {
  typedef typename EV::T TV;
  constexpr int NB = 1 << DIM;  // source 0: the tile's own chunks; nb > 0: neighbour at -(dx, dy, dz)
  // tiles in contiguous ranges per XCD, like the tile kernel's chunks, so most partials
  // are read from the L2 that wrote them (the grid may exceed the launch's tiles when it was
  // sized without the shapes; the extra workgroups exit)
  const GeoP geo = geo_of(bf);
  const uint32_t T = geo->T;
  if (geo->atomic || blockIdx.x >= T) return;
  const uint32_t t = xcd_logical_block(blockIdx.x, T, pl.xcds);
  BwdLevel lv;
  const TileCoord tc = decode_tile(pl, geo, t, &lv);
  const uint32_t bins = (uint32_t)geo->bins;
  uint32_t soff[NB], scnt[NB];
  soff[0] = bf.chunk_off[t];
  scnt[0] = bf.chunk_off[t + 1] - soff[0];
  bool single = scnt[0] == 1u;
#pragma unroll
  for (int nb = 1; nb < NB; ++nb) {
    const int dx = nb & 1, dy = (nb >> 1) & 1, dz = (nb >> 2) & 1;
    soff[nb] = 0u;
    scnt[nb] = 0u;
    if ((dx && tc.tx == 0) || (dy && tc.ty == 0) || (dz && tc.tz == 0)) continue;
    const int tibn = lv.tile_off + ((tc.tz - dz) * lv.nty + (tc.ty - dy)) * lv.ntx + (tc.tx - dx);
    const uint32_t tn = tc.g * bins + (((uint32_t)tibn << pl.hg_log2) | tc.hsub);
    soff[nb] = bf.chunk_off[tn];
    scnt[nb] = bf.chunk_off[tn + 1] - soff[nb];
    single = single && scnt[nb] == 1u;
  }
  const uint32_t nch = scnt[0];
  const size_t stride = (size_t)pl.rcells * pl.C;  // floats between chunks' partials
  TV* gv = static_cast<TV*>(bf.grad_value);
  for (int i = threadIdx.x; i < pl.cells * pl.nvec; i += kBlock) {
    const int cell = (int)fdiv((uint32_t)i, pl.div_nvec), ch = i - cell * pl.nvec;
    const int lz = (int)fdiv((uint32_t)cell, pl.div_txy), lxy = cell - lz * pl.TX * pl.TY;
    const int ly = (int)fdiv((uint32_t)lxy, pl.div_tx), lx = lxy - ly * pl.TX;
    const int x = tc.X0 + lx, y = tc.Y0 + ly, z = tc.Z0 + lz;
    if (x >= lv.W || y >= lv.H || z >= lv.D) continue;
    const bool interior = lx > 0 && ly > 0 && (DIM == 2 || lz > 0);
    if (nch == 1 && interior) continue;  // written by the tile kernel
    // each source's first partial of this cell (its region cell in that tile's layout)
    const float* src[NB];
    bool use[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int dx = nb & 1, dy = (nb >> 1) & 1, dz = (nb >> 2) & 1;
      use[nb] = scnt[nb] > 0u && (!dx || lx == 0) && (!dy || ly == 0) && (!dz || lz == 0);
      const int rn = ((lz + dz * pl.TZ) * pl.RY + (ly + dy * pl.TY)) * pl.RX + (lx + dx * pl.TX);
      src[nb] = bf.scratch + ((size_t)soff[nb] * pl.rcells + rn) * pl.C + ch * VEC;
    }
    float o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = 0.0f;
    if (single) {
      float v[NB][VEC];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        if (use[nb]) {
#pragma unroll
          for (int k = 0; k < VEC; ++k) v[nb][k] = src[nb][k];
        }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        if (use[nb]) {
#pragma unroll
          for (int k = 0; k < VEC; ++k) o[k] += v[nb][k];
        }
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        if (use[nb]) add_partials<VEC>(o, src[nb], stride, scnt[nb]);
    }
    const uint32_t row = (uint32_t)lv.start + ((uint32_t)z * lv.H + y) * lv.W + x;
    store_vec<EV, VEC>(gv + (((size_t)tc.b * pl.K + row) * pl.H + tc.h) * pl.C + ch * VEC, o);
  }
}

// ------------------------------------------------------------------ geometry
// Device-resident shapes: the geometry computed from them on the device (one thread; at
// most kMaxLevels levels).
__global__ __launch_bounds__(kWave) void bwd_geom_kernel(const GeomArgs a, const int32_t* shapes,
                                                         BwdGeom* dst) {
  if (threadIdx.x == 0) make_geom(a, shapes, dst);
}

// ------------------------------------------------------------------ dispatch
template <int DIM, typename EV, typename EC, int VEC>
hipError_t run_bwd_t(const BwdPlan& pl, const BwdGeom* host_geom, const GeomArgs* dev_args,
                     const int32_t* dev_shapes, const BwdBuffers& bf, hipStream_t s) {
  const uint32_t nbin_wg = (uint32_t)pl.groups * (uint32_t)pl.wgpg;
  const size_t hist_bytes = (size_t)pl.bins_cap * sizeof(uint32_t);
  if (nbin_wg == 0) return hipErrorInvalidValue;
  BwdGeom* geom = const_cast<BwdGeom*>(bf.geom);
  // host shapes: the first kernel (count, or the atomic kernel) gets the geometry as an
  // argument and stores it
  BwdPlan plx = pl;
  plx.geom_arg = host_geom ? 1 : 0;
  static const BwdGeom kNoGeom{};
  const BwdGeom& hg = host_geom ? *host_geom : kNoGeom;
  if (!host_geom)
    hipLaunchKernelGGL(bwd_geom_kernel, dim3(1), dim3(kWave), 0, s, *dev_args, dev_shapes, geom);
  if (pl.static_atomic || pl.fallback) {
    // fp32 sums scattered with global atomics, then rounded once; with device shapes these
    // kernels exit unless the geometry chose this path
    const uint32_t n = pl.value_bytes / (uint32_t)EV::kBytes;  // Bc * K * H * C
    uint32_t zb = (n / 4 + kBlock - 1) / kBlock;
    zb = zb < 1 ? 1 : (zb > 8192 ? 8192 : zb);
    if (n) hipLaunchKernelGGL(bwd_clear_sums_kernel, dim3(zb), dim3(kBlock), 0, s, plx, bf, n);
    hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 0, -1, true>), dim3(nbin_wg),
                       dim3(kGradThreads), 0, s, plx, bf, hg);
    uint32_t blocks = (uint32_t)((n / VEC + kBlock - 1) / kBlock);
    if (pl.fallback) {
      const uint64_t lb = (pl.grad_loc_elems + kBlock - 1) / kBlock;
      blocks = blocks > lb ? blocks : (uint32_t)(lb < 8192 ? lb : 8192);
    }
    blocks = blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks);
    hipLaunchKernelGGL((bwd_round_kernel<EV, EC, VEC>), dim3(blocks), dim3(kBlock), 0, s, pl, bf, n,
                       pl.grad_loc_elems, DIM);
    if (pl.static_atomic) return hipGetLastError();
  }
  // the plan's tile_dots is set exactly for 16-bit values
  constexpr bool kDots = EV::kBytes == 2;
  if (pl.tile_dots != (kDots ? 1 : 0)) return hipErrorInvalidValue;
  if constexpr (kDots) {
    // binned plans, 16-bit values: per-(tile, workgroup) sample counts from the coordinates
    // alone (the tile kernel forms the sample gradients)
    if (pl.P == 4 && pl.coords_aligned)
      hipLaunchKernelGGL((bwd_count_kernel<DIM, EC, 4>), dim3(nbin_wg), dim3(kBlock), hist_bytes, s, plx, bf, hg);
    else if (pl.P == 8 && pl.coords_aligned)
      hipLaunchKernelGGL((bwd_count_kernel<DIM, EC, 8>), dim3(nbin_wg), dim3(kBlock), hist_bytes, s, plx, bf, hg);
    else
      hipLaunchKernelGGL((bwd_count_kernel<DIM, EC, 0>), dim3(nbin_wg), dim3(kBlock), hist_bytes, s, plx, bf, hg);
  } else {
    // binned plans, fp32 values: sample gradients gathered per unit, with the counts
    // compile-time lane-group size for the common 16-byte lane loads of 4 or 8 lanes per unit
    if (pl.P == 4 && pl.coords_aligned && pl.lpu_log2 == 2)
      hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 4, 2>), dim3(nbin_wg), dim3(kGradThreads),
                         hist_bytes, s, plx, bf, hg);
    else if (pl.P == 4 && pl.coords_aligned && pl.lpu_log2 == 3)
      hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 4, 3>), dim3(nbin_wg), dim3(kGradThreads),
                         hist_bytes, s, plx, bf, hg);
    else if (pl.P == 8 && pl.coords_aligned && pl.lpu_log2 == 2)
      hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 8, 2>), dim3(nbin_wg), dim3(kGradThreads),
                         hist_bytes, s, plx, bf, hg);
    else if (pl.P == 8 && pl.coords_aligned && pl.lpu_log2 == 3)
      hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 8, 3>), dim3(nbin_wg), dim3(kGradThreads),
                         hist_bytes, s, plx, bf, hg);
    else if (pl.P == 4 && pl.coords_aligned)
      hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 4, -1>), dim3(nbin_wg), dim3(kGradThreads),
                         hist_bytes, s, plx, bf, hg);
    else if (pl.P == 8 && pl.coords_aligned)
      hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 8, -1>), dim3(nbin_wg), dim3(kGradThreads),
                         hist_bytes, s, plx, bf, hg);
    else
      hipLaunchKernelGGL((bwd_grad_kernel<DIM, EV, EC, VEC, 0, -1>), dim3(nbin_wg), dim3(kGradThreads),
                         hist_bytes, s, plx, bf, hg);
  }
  if (pl.T_cap == 0) return hipGetLastError();  // no cell in any level: grad_value is empty
  // grids sized by T_cap (the launch's tiles when the host knows the shapes, an upper bound
  // otherwise); workgroups beyond the geometry's T exit
  const uint32_t waves_per_block = kBlock / kWave;
  hipLaunchKernelGGL(bwd_colscan_kernel, dim3((pl.T_cap + waves_per_block - 1) / waves_per_block),
                     dim3(kBlock), 0, s, pl, bf);
  hipLaunchKernelGGL(bwd_plan_kernel, dim3(pl.groups), dim3(kPlanThreads), 0, s, pl, bf);
  const size_t fill_bytes = 2 * hist_bytes +
                            (size_t)kFillStage * (rec_words<DIM, EC>() + 1) * sizeof(uint32_t) +
                            (kBlock / kWave) * sizeof(uint32_t);
  if (pl.P == 4 && pl.coords_aligned)
    hipLaunchKernelGGL((bwd_fill_kernel<DIM, EC, 4>), dim3(nbin_wg), dim3(kBlock), fill_bytes, s, pl, bf);
  else if (pl.P == 8 && pl.coords_aligned)
    hipLaunchKernelGGL((bwd_fill_kernel<DIM, EC, 8>), dim3(nbin_wg), dim3(kBlock), fill_bytes, s, pl, bf);
  else
    hipLaunchKernelGGL((bwd_fill_kernel<DIM, EC, 0>), dim3(nbin_wg), dim3(kBlock), fill_bytes, s, pl, bf);
  hipLaunchKernelGGL((bwd_tile_kernel<DIM, EV, EC, VEC, kDots>), dim3(pl.grid_chunks),
                     dim3(kTileThreads<DIM>), pl.lds_bytes, s, pl, bf);
  hipLaunchKernelGGL((bwd_fold_kernel<DIM, EV, VEC>), dim3(pl.T_cap), dim3(kBlock), 0, s, pl, bf);
  return hipGetLastError();
}

using BwdFn = hipError_t (*)(const BwdPlan&, const BwdGeom*, const GeomArgs*, const int32_t*,
                             const BwdBuffers&, hipStream_t);

template <int DIM, typename EV, typename EC>
BwdFn pick_vec(int vec_bytes) {
  constexpr int S = EV::kBytes;
  switch (vec_bytes) {
    case 16: return &run_bwd_t<DIM, EV, EC, 16 / S>;
    case 8: return &run_bwd_t<DIM, EV, EC, 8 / S>;
    case 4: return &run_bwd_t<DIM, EV, EC, 4 / S>;
    case 2:
      if constexpr (S == 2) return &run_bwd_t<DIM, EV, EC, 1>;
      return nullptr;
    default: return nullptr;
  }
}

template <int DIM>
BwdFn pick_types(int vdt, int cdt, int vec_bytes) {
  if (vdt == 0 && cdt == 0) return pick_vec<DIM, F32, F32>(vec_bytes);
  if (vdt == 1 && cdt == 1) return pick_vec<DIM, F16, F16>(vec_bytes);
  if (vdt == 1 && cdt == 0) return pick_vec<DIM, F16, F32>(vec_bytes);
  if (vdt == 2 && cdt == 2) return pick_vec<DIM, BF16, BF16>(vec_bytes);
  if (vdt == 2 && cdt == 0) return pick_vec<DIM, BF16, F32>(vec_bytes);
  return nullptr;
}

BwdFn get_bwd(int dim, int vdt, int cdt, int vec_bytes) {
  if (dim == 2) return pick_types<2>(vdt, cdt, vec_bytes);
  if (dim == 3) return pick_types<3>(vdt, cdt, vec_bytes);
  return nullptr;
}

}  // namespace

__global__ __launch_bounds__(kBlock) void zero_bytes_kernel(uint8_t* p, size_t n, int vec) {
  const size_t n16 = vec ? n / 16 : 0;
  const size_t stride = (size_t)gridDim.x * kBlock;
  const size_t t0 = (size_t)blockIdx.x * kBlock + threadIdx.x;
  for (size_t i = t0; i < n16; i += stride) reinterpret_cast<u32x4*>(p)[i] = u32x4{0u, 0u, 0u, 0u};
  for (size_t i = n16 * 16 + t0; i < n; i += stride) p[i] = 0;
}

hipError_t launch_zero_bytes(void* p, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  size_t blocks = (bytes / 16 + kBlock - 1) / kBlock;
  blocks = blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks);
  const int vec = ((uintptr_t)p % 16) == 0;
  hipLaunchKernelGGL(zero_bytes_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s,
                     static_cast<uint8_t*>(p), bytes, vec);
  return hipGetLastError();
}

bool bwd_supported(int dim, int vdt, int cdt, int vec_bytes) {
  return get_bwd(dim, vdt, cdt, vec_bytes) != nullptr;
}

BwdSizes bwd_sizes(const BwdPlan& pl, uint64_t samples, int dim, int coord_bytes) {
  BwdSizes z;
  const bool binned = !pl.static_atomic;
  const bool sums = pl.static_atomic || pl.fallback;
  z.counts = binned ? (uint64_t)pl.groups * pl.wgpg * pl.bins_cap : 0u;
  z.tile_n = (uint64_t)pl.T_cap + 1;
  z.bin_start = (uint64_t)pl.T_cap + 1;
  z.chunk_off = (uint64_t)pl.T_cap + 1;
  z.chunk_words = (uint64_t)pl.max_chunks * 4u;
  z.record_words = binned ? (samples > 0 ? samples : 1) * (uint64_t)record_words(dim, coord_bytes) : 0u;
  z.scratch_floats = binned ? (uint64_t)pl.max_chunks * pl.rcells * pl.C : 0u;
  // atomic path: one fp32 sum per grad_value element of a launch (groups << hg_log2 =
  // batches * H)
  z.sum_floats = sums ? ((uint64_t)pl.groups << pl.hg_log2) * (uint64_t)pl.K * pl.C : 0u;
  z.geom_bytes = sizeof(BwdGeom);
  auto al = [](uint64_t b) { return (b + 255) & ~(uint64_t)255; };
  z.total_bytes = al(z.counts * 4) + al(z.tile_n * 4) + al(z.bin_start * 4) + al(z.chunk_off * 4) +
                  al(z.chunk_words * 4) + al(z.record_words * 4) + al(z.scratch_floats * 4) +
                  al(z.sum_floats * 4) + al(z.geom_bytes);
  return z;
}

hipError_t run_bwd(const BwdPlan& pl, const BwdGeom* host_geom, const GeomArgs* dev_args,
                   const int32_t* dev_shapes, const BwdBuffers& bf, int dim, int vdt, int cdt,
                   int vec_bytes, hipStream_t s) {
  BwdFn fn = get_bwd(dim, vdt, cdt, vec_bytes);
  if (!fn || (!host_geom && (!dev_args || !dev_shapes))) return hipErrorInvalidValue;
  return fn(pl, host_geom, dev_args, dev_shapes, bf, s);
}

}  // namespace msda
