// msda_bwd.hip — gfx950 backward of multi-scale deformable attention without global
// floating-point atomics.
//
// Replaces the reference's _bwd_kernel_2d (src/msda_triton/triton/msda_2d.py:263-510) and
// 3D _bwd_kernel (src/msda_triton/triton/msda_3d.py:291-653), which scatter grad_value
// with one global atomic per (sample, corner, channel). On MI355X global fp32 atomics on
// random rows sustain about 0.33 T element-adds/s and LDS fp32 atomics about a third of
// an operation per clock per CU, so this backward accumulates grad_value in key order:
//
//  1. bin count: every sample with a valid corner is assigned to the tile of its level
//     that owns its lowest corner. Each workgroup covers the units of one (batch,
//     head-group), histograms its samples per tile in LDS (integer atomics, full rate),
//     and writes the histogram as one row of a per-(workgroup, tile) count matrix.
//  2. column scan: per tile, the counts of all workgroups become offsets within the tile
//     and the tile's total.
//  3. plan (one workgroup): exclusive scan of the tile totals, chunks of at most R records
//     per tile, and the chunk -> tile table.
//  4. bin fill: the same traversal writes each sample's record (id, clamp flags, pixel
//     coordinates, attention weight) at its tile's base + offset + LDS rank, so later
//     passes never re-read locations or weights at random addresses.
//  5. tile kernel: one workgroup per chunk, chunks of one (batch, head-group) on one XCD.
//     It stages the tile's value region (tile + one-cell high-side halo) in LDS; per
//     sub-batch of S records it stages grad_out rows, forms <grad_out, value_corner> from
//     the staged rows and stores grad_attention_weights and grad_sampling_locations,
//     sorts the (corner weight * attn, record) entries by region cell, and accumulates
//     grad_value for every region cell in the fp32 registers of the cell's owner threads.
//     Interior cells of a one-chunk tile are written directly in the value dtype; edge
//     cells (which also receive halo contributions of lower neighbours), halo cells and
//     every cell of a split tile are written as fp32 partials.
//  6. fold: per tile, sums the partials of its own chunks and the halo partials of its
//     lower neighbours' chunks, in a fixed order, and writes the edge / split cells.
//
// Every grad_value element is written exactly once with a plain store, so no clearing
// pass is needed and 16-bit values are rounded once, from fp32.
#include "msda_internal.h"
#include "msda_sample.h"

namespace msda {

namespace {

constexpr int kPlanThreads = 1024;

// ------------------------------------------------------------------ block scans
__device__ inline uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t t = __shfl_up(v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

// Exclusive scan of one value per thread across a workgroup of NT threads; *total gets
// the sum. s_w holds NT / 64 words. Every thread of the workgroup must call it.
template <int NT>
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* s_w, uint32_t* total) {
  const uint32_t inc = wave_incl_scan(v);
  const int w = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  if (lane == kWave - 1) s_w[w] = inc;
  __syncthreads();
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / kWave; ++i) {
    const uint32_t x = s_w[i];
    if (i < w) pre += x;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return pre + inc - v;
}

// ------------------------------------------------------------------ tiles
struct TileCoord {
  uint32_t g, hsub, b, h;
  int l, tx, ty, tz, X0, Y0, Z0;
};

__device__ inline TileCoord decode_tile(const BwdPlan& pl, uint32_t t) {
  TileCoord tc;
  tc.g = t / (uint32_t)pl.bins;
  const uint32_t bin = t - tc.g * (uint32_t)pl.bins;
  tc.hsub = bin / (uint32_t)pl.tiles_per_bh;
  const int tib = (int)(bin - tc.hsub * (uint32_t)pl.tiles_per_bh);
  const uint32_t gph = (uint32_t)pl.H >> pl.hg_log2;
  tc.b = tc.g / gph;
  tc.h = ((tc.g - tc.b * gph) << pl.hg_log2) | tc.hsub;
  int l = 0;
  while (l + 1 < pl.L && pl.lv[l + 1].tile_off <= tib) ++l;
  tc.l = l;
  const BwdLevel& lv = pl.lv[l];
  const int lt = tib - lv.tile_off;
  tc.tx = lt % lv.ntx;
  tc.ty = (lt / lv.ntx) % lv.nty;
  tc.tz = lt / (lv.ntx * lv.nty);
  tc.X0 = tc.tx * pl.TX;
  tc.Y0 = tc.ty * pl.TY;
  tc.Z0 = tc.tz * pl.TZ;
  return tc;
}

// Region-cell index of a corner relative to the tile origin, or -1 outside the region.
__device__ inline int region_cell(const BwdPlan& pl, int ox, int oy, int oz) {
  if ((unsigned)ox >= (unsigned)pl.RX || (unsigned)oy >= (unsigned)pl.RY ||
      (unsigned)oz >= (unsigned)pl.RZ)
    return -1;
  return (oz * pl.RY + oy) * pl.RX + ox;
}

// ------------------------------------------------------------------ 1, 4: binning
// One thread per unit (b, q, h) of a (batch, head-group): u = w * kBlock + tid enumerates
// (q, head-in-group). FILL = false counts samples per tile; FILL = true writes records.
template <int DIM, typename EC, bool FILL>
__global__ __launch_bounds__(kBlock) void bwd_bin_kernel(const BwdPlan pl, const BwdBuffers bf) {
  typedef typename EC::T TC;
  extern __shared__ uint32_t s_hist[];  // [bins] counters, then [bins] record bases (fill)
  uint32_t* s_base = s_hist + pl.bins;
  const uint32_t g = blockIdx.x / (uint32_t)pl.wgpg;
  const uint32_t w = blockIdx.x - g * (uint32_t)pl.wgpg;
  const size_t crow = ((size_t)g * pl.wgpg + w) * pl.bins;
  for (int i = threadIdx.x; i < pl.bins; i += kBlock) {
    s_hist[i] = 0;
    if (FILL) s_base[i] = bf.bin_start[(size_t)g * pl.bins + i] + bf.counts[crow + i];
  }
  __syncthreads();

  const uint32_t HG = 1u << pl.hg_log2;
  const uint32_t u = w * kBlock + threadIdx.x;
  if (u < pl.Q * HG) {
    const uint32_t q = u >> pl.hg_log2, hsub = u & (HG - 1u);
    const uint32_t gph = (uint32_t)pl.H >> pl.hg_log2;
    const uint32_t b = g / gph, h = ((g - b * gph) << pl.hg_log2) | hsub;
    const int LP = pl.L * pl.P;
    const size_t bqh = ((size_t)b * pl.Q + q) * pl.H + h;
    const TC* locp = static_cast<const TC*>(bf.loc) + bqh * LP * DIM;
    const TC* attp = static_cast<const TC*>(bf.attn) + bqh * LP;
    for (int l = 0; l < pl.L; ++l) {
      const BwdLevel& lv = pl.lv[l];
      for (int p = 0; p < pl.P; ++p) {
        const int s = l * pl.P + p;
        bool px, py, pz = true;
        const float ux = grid_to_u((float)locp[s * DIM + 0], (float)lv.W, pl.clamp, pl.lo_g, pl.hi_g, &px);
        const float uy = grid_to_u((float)locp[s * DIM + 1], (float)lv.H, pl.clamp, pl.lo_g, pl.hi_g, &py);
        float uz = 0.0f;
        if constexpr (DIM == 3)
          uz = grid_to_u((float)locp[s * DIM + 2], (float)lv.D, pl.clamp, pl.lo_g, pl.hi_g, &pz);
        const Axis ax = axis_from_u(ux, lv.W, px);
        const Axis ay = axis_from_u(uy, lv.H, py);
        const Axis az = DIM == 3 ? axis_from_u(uz, lv.D, pz) : Axis{1.0f, 0.0f, 0, true, false, true};
        if (!(ax.v0 || ax.v1) || !(ay.v0 || ay.v1) || !(az.v0 || az.v1)) {
          // no corner inside the level: the sample's gradients are zero
          if (!FILL) {
            TC* gl = static_cast<TC*>(bf.grad_loc) + (bqh * LP + s) * DIM;
#pragma unroll
            for (int d = 0; d < DIM; ++d) gl[d] = (TC)0.0f;
            static_cast<TC*>(bf.grad_attn)[bqh * LP + s] = (TC)0.0f;
          }
          continue;
        }
        const int tx = anchor_tile(ax, pl.TX), ty = anchor_tile(ay, pl.TY);
        const int tz = DIM == 3 ? anchor_tile(az, pl.TZ) : 0;
        const int tib = lv.tile_off + (tz * lv.nty + ty) * lv.ntx + tx;
        const uint32_t bin = hsub * (uint32_t)pl.tiles_per_bh + (uint32_t)tib;
        const uint32_t r = atomicAdd(&s_hist[bin], 1u);
        if (FILL) {
          const uint32_t id = (q * (uint32_t)pl.P + (uint32_t)p) | (px ? kRecPassX : 0u) |
                              (py ? kRecPassY : 0u) | (pz ? kRecPassZ : 0u);
          const float a = (float)attp[s];
          uint32_t* rec = bf.records + (size_t)(s_base[bin] + r) * (DIM + 2);
          if constexpr (DIM == 2) {
            *reinterpret_cast<u32x4*>(rec) =
                u32x4{id, __builtin_bit_cast(uint32_t, ux), __builtin_bit_cast(uint32_t, uy),
                      __builtin_bit_cast(uint32_t, a)};
          } else {
            rec[0] = id;
            rec[1] = __builtin_bit_cast(uint32_t, ux);
            rec[2] = __builtin_bit_cast(uint32_t, uy);
            rec[3] = __builtin_bit_cast(uint32_t, uz);
            rec[4] = __builtin_bit_cast(uint32_t, a);
          }
        }
      }
    }
  }
  if (!FILL) {
    __syncthreads();
    for (int i = threadIdx.x; i < pl.bins; i += kBlock) bf.counts[crow + i] = s_hist[i];
  }
}

// ------------------------------------------------------------------ 2: column scan
// One thread per tile: the tile's counts over the bin workgroups of its group become
// offsets within the tile, and its total goes to bin_start[t].
__global__ __launch_bounds__(kBlock) void bwd_colscan_kernel(const BwdPlan pl, const BwdBuffers bf) {
  const uint32_t t = blockIdx.x * kBlock + threadIdx.x;
  if (t >= pl.T) return;
  const uint32_t g = t / (uint32_t)pl.bins, i = t - g * (uint32_t)pl.bins;
  uint32_t run = 0;
  for (int w = 0; w < pl.wgpg; ++w) {
    const size_t idx = ((size_t)g * pl.wgpg + w) * pl.bins + i;
    const uint32_t c = bf.counts[idx];
    bf.counts[idx] = run;
    run += c;
  }
  bf.bin_start[t] = run;
}

// ------------------------------------------------------------------ 3: plan
// One workgroup. Each thread owns a contiguous range of tiles: scans record totals into
// first-record offsets, cuts each tile into max(1, ceil(n / R)) chunks (an empty tile
// still gets one chunk, which writes its zeros), and fills the chunk -> tile table.
__global__ __launch_bounds__(kPlanThreads) void bwd_plan_kernel(const BwdPlan pl, const BwdBuffers bf) {
  __shared__ uint32_t s_w[kPlanThreads / kWave];
  const uint32_t per = (pl.T + kPlanThreads - 1) / kPlanThreads;
  const uint32_t t0 = min(pl.T, threadIdx.x * per), t1 = min(pl.T, t0 + per);
  uint32_t sn = 0, sc = 0;
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t n = bf.bin_start[t];
    sn += n;
    sc += max(1u, (n + pl.R - 1) / pl.R);
  }
  uint32_t tot_n, tot_c;
  uint32_t pn = block_excl_scan<kPlanThreads>(sn, s_w, &tot_n);
  uint32_t pc = block_excl_scan<kPlanThreads>(sc, s_w, &tot_c);
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t n = bf.bin_start[t];
    const uint32_t nch = max(1u, (n + pl.R - 1) / pl.R);
    bf.bin_start[t] = pn;
    bf.chunk_off[t] = pc;
    for (uint32_t k = 0; k < nch; ++k) bf.chunk_tile[pc + k] = t;
    pn += n;
    pc += nch;
  }
  if (threadIdx.x == 0) {
    bf.bin_start[pl.T] = tot_n;
    bf.chunk_off[pl.T] = tot_c;
  }
}

// Axes of a staged record.
template <int DIM>
__device__ inline Sample<DIM> record_sample(const uint32_t* rec, const BwdLevel& lv) {
  Sample<DIM> sm;
  const uint32_t id = rec[0];
  sm.ax = axis_from_u(__builtin_bit_cast(float, rec[1]), lv.W, (id & kRecPassX) != 0);
  sm.ay = axis_from_u(__builtin_bit_cast(float, rec[2]), lv.H, (id & kRecPassY) != 0);
  if constexpr (DIM == 3) sm.az = axis_from_u(__builtin_bit_cast(float, rec[3]), lv.D, (id & kRecPassZ) != 0);
  return sm;
}

// ------------------------------------------------------------------ 5: tile kernel
// One workgroup (kTileThreads threads) per chunk of a tile's records. LDS holds the staged
// value region, and per sub-batch of up to S records: each record's grad_out row, the
// record itself, the (weight, record) entries of its corners sorted by region cell, and
// per-cell counters. Per sub-batch:
//   A. record pass (2^lpu_log2 lanes per record): stage the record and its grad_out row;
//      form <grad_out, value_corner> from the staged value rows and store
//      grad_attention_weights / grad_sampling_locations; count corners per region cell.
//   B. exclusive scan of the per-cell counts.
//   C. entry pass (one thread per record): place (attn * w_corner, record) entries of the
//      record's corners at their cell's offset + rank.
//   D. owner pass: the thread owning (region cell, channel chunk) sums attn*w*grad_out over
//      its cell's entries in fp32 registers.
template <int DIM, typename EV, typename EC, int VEC>
__global__ __launch_bounds__(kTileThreads) void bwd_tile_kernel(const BwdPlan pl,
                                                                const BwdBuffers bf) {
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  constexpr int RW = DIM + 2;        // words per record
  constexpr int MI = kTileMaxItems;  // owner items per thread
  typedef typename EC::T TC;
  typedef typename EV::T TV;
  extern __shared__ __attribute__((aligned(16))) char s_mem[];

  // Chunks are dealt to XCDs in contiguous ranges (workgroup i runs on XCD i % 8), so the
  // chunks of one (batch, head-group) share an XCD and its L2.
  const uint32_t total = bf.chunk_off[pl.T];
  const uint32_t per = (total + kXcds - 1) / kXcds;
  const uint32_t slot = blockIdx.x / kXcds;
  if (slot >= per) return;
  const uint32_t c = (blockIdx.x % kXcds) * per + slot;
  if (c >= total) return;  // the whole workgroup exits
  const uint32_t t = bf.chunk_tile[c];
  const uint32_t off = bf.chunk_off[t];
  const uint32_t nch = bf.chunk_off[t + 1] - off;
  const uint32_t beg = bf.bin_start[t] + (c - off) * pl.R;
  const uint32_t end = min(bf.bin_start[t + 1], beg + pl.R);
  const TileCoord tc = decode_tile(pl, t);
  const BwdLevel lv = pl.lv[tc.l];

  char* s_val = s_mem;
  char* s_g = s_mem + pl.lds_val_bytes;                                      // [S][C] raw rows
  uint2* s_ent = reinterpret_cast<uint2*>(s_g + pl.lds_g_bytes);             // [S * NC]
  uint32_t* s_rec = reinterpret_cast<uint32_t*>(s_ent + (size_t)pl.S * NC);  // [S][RW]
  uint32_t* s_cnt = s_rec + (size_t)pl.S * RW;                               // [rcells + 1]
  uint32_t* s_cur = s_cnt + pl.rcells + 1;                                   // [rcells]
  uint32_t* s_w = s_cur + pl.rcells;                                         // [waves]
  const int ncell_r = pl.rcells;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(bf.value, pl.value_bytes);
  const uint32_t rs = (uint32_t)pl.H * (uint32_t)pl.C * EV::kBytes;  // bytes between rows of K
  const uint32_t bh_base = ((tc.b * (uint32_t)pl.K) * (uint32_t)pl.H + tc.h) * (uint32_t)pl.C * EV::kBytes;
  const uint32_t grow = (uint32_t)pl.C * EV::kBytes;  // bytes of one staged grad_out row
  const int LP = pl.L * pl.P;

  // stage the value region [X0, X0+TX] x [Y0, Y0+TY] (x [Z0, Z0+TZ]); cells outside the
  // level read as zero
  for (int i = threadIdx.x; i < ncell_r * pl.nvec; i += kTileThreads) {
    const int cell = i / pl.nvec, ch = i - cell * pl.nvec;
    const int rx = cell % pl.RX, ry = (cell / pl.RX) % pl.RY, rz = cell / (pl.RX * pl.RY);
    const int x = tc.X0 + rx, y = tc.Y0 + ry, z = tc.Z0 + rz;
    const bool in = x < lv.W && y < lv.H && z < lv.D;
    const uint32_t row = (uint32_t)lv.start + ((uint32_t)z * lv.H + y) * lv.W + x;
    const RawVec<VB> r = buf_load<VB>(rv, in ? bh_base + row * rs + ch * VB : kOobOffset);
    *reinterpret_cast<RawVec<VB>*>(s_val + cell * pl.val_row_bytes + ch * VB) = r;
  }

  float acc[MI][VEC];
#pragma unroll
  for (int m = 0; m < MI; ++m)
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[m][k] = 0.0f;

  const int lg = pl.lpu_log2;
  const uint32_t lanes = 1u << lg;
  const uint32_t grp = threadIdx.x >> lg;
  const uint32_t lane = threadIdx.x & (lanes - 1u);
  const bool act = (int)lane < pl.nvec;
  const uint32_t groups = (uint32_t)kTileThreads >> lg;

  for (uint32_t sb = beg; sb < end; sb += pl.S) {
    const uint32_t nrec = min((uint32_t)pl.S, end - sb);
    for (int i = threadIdx.x; i <= ncell_r; i += kTileThreads) s_cnt[i] = 0u;
    __syncthreads();  // value region staged (first sub-batch); counters cleared

    // A. record pass
    for (uint32_t r = grp; r < nrec; r += groups) {
      uint32_t rw[RW];
      const uint32_t* grec = bf.records + (size_t)(sb + r) * RW;
#pragma unroll
      for (int k = 0; k < RW; ++k) rw[k] = grec[k];
      if (lane == 0) {
#pragma unroll
        for (int k = 0; k < RW; ++k) s_rec[r * RW + k] = rw[k];
      }
      const uint32_t qp = rw[0] & kRecIdMask;
      const uint32_t q = fdiv(qp, pl.div_p), p = qp - q * (uint32_t)pl.P;
      const size_t bqh = ((size_t)tc.b * pl.Q + q) * pl.H + tc.h;
      const size_t si = bqh * LP + (size_t)tc.l * pl.P + p;
      const Sample<DIM> sm = record_sample<DIM>(rw, lv);
      float g[VEC];
      if (act) {
        const RawVec<VB> raw =
            glb_load<VB>(static_cast<const TV*>(bf.grad_out) + bqh * pl.C + lane * VEC);
        *reinterpret_cast<RawVec<VB>*>(s_g + r * grow + lane * VB) = raw;
        widen<EV, VEC>(raw, g);
      } else {
#pragma unroll
        for (int k = 0; k < VEC; ++k) g[k] = 0.0f;
      }
      // count the valid corners per region cell, one lane per corner
      for (int cc = (int)lane; cc < NC; cc += (int)lanes) {
        const int cell = region_cell(pl, sm.ax.i0 + (cc & 1) - tc.X0, sm.ay.i0 + ((cc >> 1) & 1) - tc.Y0,
                                     DIM == 3 ? sm.az.i0 + ((cc >> 2) & 1) - tc.Z0 : 0);
        if (corner_valid<DIM>(cc, sm) && cell >= 0) atomicAdd(&s_cnt[cell], 1u);
      }
      float dot[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const int cell = region_cell(pl, sm.ax.i0 + (cc & 1) - tc.X0, sm.ay.i0 + ((cc >> 1) & 1) - tc.Y0,
                                     DIM == 3 ? sm.az.i0 + ((cc >> 2) & 1) - tc.Z0 : 0);
        dot[cc] = 0.0f;
        if (act && corner_valid<DIM>(cc, sm) && cell >= 0) {
          const RawVec<VB> rwv =
              *reinterpret_cast<const RawVec<VB>*>(s_val + cell * pl.val_row_bytes + lane * VB);
          float v[VEC];
          widen<EV, VEC>(rwv, v);
          float d = 0.0f;
#pragma unroll
          for (int k = 0; k < VEC; ++k) d = __builtin_fmaf(g[k], v[k], d);
          dot[cc] = d;
        }
      }
      float s_attn, s_x, s_y, s_z;
      corner_grads<DIM>(sm, dot, s_attn, s_x, s_y, s_z);
      s_attn = group_sum(s_attn, lg);
      s_x = group_sum(s_x, lg);
      s_y = group_sum(s_y, lg);
      if constexpr (DIM == 3) s_z = group_sum(s_z, lg);
      if (lane == 0) {
        const float a = __builtin_bit_cast(float, rw[RW - 1]);
        static_cast<TC*>(bf.grad_attn)[si] = (TC)s_attn;
        TC* gl = static_cast<TC*>(bf.grad_loc) + si * DIM;
        gl[0] = (TC)(sm.ax.pass ? (a * s_x) * (float)lv.W : 0.0f);
        gl[1] = (TC)(sm.ay.pass ? (a * s_y) * (float)lv.H : 0.0f);
        if constexpr (DIM == 3) gl[2] = (TC)(sm.az.pass ? (a * s_z) * (float)lv.D : 0.0f);
      }
    }
    __syncthreads();

    // B. exclusive scan of the per-cell counts (rcells <= kTileThreads)
    {
      const uint32_t v = (int)threadIdx.x < ncell_r ? s_cnt[threadIdx.x] : 0u;
      uint32_t tot;
      const uint32_t ex = block_excl_scan<kTileThreads>(v, s_w, &tot);
      if ((int)threadIdx.x < ncell_r) {
        s_cnt[threadIdx.x] = ex;
        s_cur[threadIdx.x] = 0u;
      }
      if (threadIdx.x == 0) s_cnt[ncell_r] = tot;
    }
    __syncthreads();

    // C. entry pass: one thread per record
    for (uint32_t r = threadIdx.x; r < nrec; r += kTileThreads) {
      const uint32_t* rw = s_rec + r * RW;
      const Sample<DIM> sm = record_sample<DIM>(rw, lv);
      const float a = __builtin_bit_cast(float, rw[RW - 1]);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const int cell = region_cell(pl, sm.ax.i0 + (cc & 1) - tc.X0, sm.ay.i0 + ((cc >> 1) & 1) - tc.Y0,
                                     DIM == 3 ? sm.az.i0 + ((cc >> 2) & 1) - tc.Z0 : 0);
        if (corner_valid<DIM>(cc, sm) && cell >= 0) {
          const uint32_t pos = s_cnt[cell] + atomicAdd(&s_cur[cell], 1u);
          const float cw = corner_weight<DIM>(cc, sm) * a;
          s_ent[pos] = make_uint2(__builtin_bit_cast(uint32_t, cw), r);
        }
      }
    }
    __syncthreads();

    // D. owner pass: fp32 register accumulation per (region cell, channel chunk)
#pragma unroll
    for (int m = 0; m < MI; ++m) {
      const int it = (int)threadIdx.x + m * kTileThreads;
      if (it < ncell_r * pl.nvec) {
        const int cell = it / pl.nvec, ch = it - cell * pl.nvec;
        const uint32_t e0 = s_cnt[cell], e1 = s_cnt[cell + 1];
        for (uint32_t e = e0; e < e1; ++e) {
          const uint2 en = s_ent[e];
          const float cw = __builtin_bit_cast(float, en.x);
          const RawVec<VB> raw = *reinterpret_cast<const RawVec<VB>*>(s_g + en.y * grow + ch * VB);
          float gv[VEC];
          widen<EV, VEC>(raw, gv);
#pragma unroll
          for (int k = 0; k < VEC; ++k) acc[m][k] = __builtin_fmaf(cw, gv[k], acc[m][k]);
        }
      }
    }
    __syncthreads();  // LDS of this sub-batch is reused by the next one
  }

  // write the region: interior cells of a one-chunk tile directly in the value dtype;
  // edge cells, halo cells inside the level and all cells of a split tile as fp32 partials
  // for the fold kernel
#pragma unroll
  for (int m = 0; m < MI; ++m) {
    const int it = (int)threadIdx.x + m * kTileThreads;
    if (it >= ncell_r * pl.nvec) continue;
    const int cell = it / pl.nvec, ch = it - cell * pl.nvec;
    const int rx = cell % pl.RX, ry = (cell / pl.RX) % pl.RY, rz = cell / (pl.RX * pl.RY);
    const int x = tc.X0 + rx, y = tc.Y0 + ry, z = tc.Z0 + rz;
    if (x >= lv.W || y >= lv.H || z >= lv.D) continue;
    const bool owned = rx < pl.TX && ry < pl.TY && rz < pl.TZ;
    const bool interior = owned && rx > 0 && ry > 0 && (DIM == 2 || rz > 0);
    if (nch == 1 && interior) {
      const uint32_t row = (uint32_t)lv.start + ((uint32_t)z * lv.H + y) * lv.W + x;
      store_vec<EV, VEC>(static_cast<TV*>(bf.grad_value) +
                             (((size_t)tc.b * pl.K + row) * pl.H + tc.h) * pl.C + ch * VEC,
                         acc[m]);
    } else {
      float* dst = bf.scratch + ((size_t)c * ncell_r + cell) * pl.C + ch * VEC;
#pragma unroll
      for (int k = 0; k < VEC; ++k) dst[k] = acc[m][k];
    }
  }
}

// ------------------------------------------------------------------ 6: fold
// One workgroup per tile. Sums, for every edge cell (and every cell of a split tile), the
// partials of the tile's own chunks and then the halo partials of the chunks of the lower
// neighbours whose halo covers the cell, and writes the cell in the value dtype.
template <int DIM, typename EV, int VEC>
__global__ __launch_bounds__(kBlock) void bwd_fold_kernel(const BwdPlan pl, const BwdBuffers bf) {
  typedef typename EV::T TV;
  const uint32_t t = blockIdx.x;
  const uint32_t off = bf.chunk_off[t];
  const uint32_t nch = bf.chunk_off[t + 1] - off;
  const TileCoord tc = decode_tile(pl, t);
  const BwdLevel lv = pl.lv[tc.l];
  const uint32_t tbase = t - (uint32_t)((tc.tz * lv.nty + tc.ty) * lv.ntx + tc.tx);
  TV* gv = static_cast<TV*>(bf.grad_value);
  for (int i = threadIdx.x; i < pl.cells * pl.nvec; i += kBlock) {
    const int cell = i / pl.nvec, ch = i - cell * pl.nvec;
    const int lx = cell % pl.TX, ly = (cell / pl.TX) % pl.TY, lz = cell / (pl.TX * pl.TY);
    const int x = tc.X0 + lx, y = tc.Y0 + ly, z = tc.Z0 + lz;
    if (x >= lv.W || y >= lv.H || z >= lv.D) continue;
    const bool interior = lx > 0 && ly > 0 && (DIM == 2 || lz > 0);
    if (nch == 1 && interior) continue;  // written by the tile kernel
    float o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = 0.0f;
    const int rc = (lz * pl.RY + ly) * pl.RX + lx;
    for (uint32_t j = 0; j < nch; ++j) {
      const float* src = bf.scratch + ((size_t)(off + j) * pl.rcells + rc) * pl.C + ch * VEC;
#pragma unroll
      for (int k = 0; k < VEC; ++k) o[k] += src[k];
    }
    for (int nb = 1; nb < (1 << DIM); ++nb) {
      const int dx = nb & 1, dy = (nb >> 1) & 1, dz = (nb >> 2) & 1;
      if ((dx && (lx != 0 || tc.tx == 0)) || (dy && (ly != 0 || tc.ty == 0)) ||
          (dz && (lz != 0 || tc.tz == 0)))
        continue;
      const uint32_t tn = tbase + (uint32_t)(((tc.tz - dz) * lv.nty + (tc.ty - dy)) * lv.ntx + (tc.tx - dx));
      const int rn = ((lz + dz * pl.TZ) * pl.RY + (ly + dy * pl.TY)) * pl.RX + (lx + dx * pl.TX);
      const uint32_t noff = bf.chunk_off[tn], nn = bf.chunk_off[tn + 1] - noff;
      for (uint32_t j = 0; j < nn; ++j) {
        const float* src = bf.scratch + ((size_t)(noff + j) * pl.rcells + rn) * pl.C + ch * VEC;
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[k] += src[k];
      }
    }
    const uint32_t row = (uint32_t)lv.start + ((uint32_t)z * lv.H + y) * lv.W + x;
    store_vec<EV, VEC>(gv + (((size_t)tc.b * pl.K + row) * pl.H + tc.h) * pl.C + ch * VEC, o);
  }
}

// ------------------------------------------------------------------ dispatch
template <int DIM, typename EV, typename EC, int VEC>
hipError_t run_bwd_t(const BwdPlan& pl, const BwdBuffers& bf, hipStream_t s) {
  const uint32_t nbin_wg = (uint32_t)pl.groups * (uint32_t)pl.wgpg;
  const size_t hist_bytes = (size_t)pl.bins * sizeof(uint32_t);
  if (nbin_wg == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL((bwd_bin_kernel<DIM, EC, false>), dim3(nbin_wg), dim3(kBlock), hist_bytes, s,
                     pl, bf);
  if (pl.T == 0) return hipGetLastError();  // no cell in any level: grad_value is empty
  hipLaunchKernelGGL(bwd_colscan_kernel, dim3((pl.T + kBlock - 1) / kBlock), dim3(kBlock), 0, s,
                     pl, bf);
  hipLaunchKernelGGL(bwd_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, pl, bf);
  hipLaunchKernelGGL((bwd_bin_kernel<DIM, EC, true>), dim3(nbin_wg), dim3(kBlock), 2 * hist_bytes,
                     s, pl, bf);
  hipLaunchKernelGGL((bwd_tile_kernel<DIM, EV, EC, VEC>), dim3(pl.grid_chunks),
                     dim3(kTileThreads), pl.lds_bytes, s, pl, bf);
  hipLaunchKernelGGL((bwd_fold_kernel<DIM, EV, VEC>), dim3(pl.T), dim3(kBlock), 0, s, pl, bf);
  return hipGetLastError();
}

using BwdFn = hipError_t (*)(const BwdPlan&, const BwdBuffers&, hipStream_t);

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

BwdSizes bwd_sizes(const BwdPlan& pl, uint64_t samples, int dim) {
  BwdSizes z;
  z.counts = (uint64_t)pl.groups * pl.wgpg * pl.bins;
  z.bin_start = (uint64_t)pl.T + 1;
  z.chunk_off = (uint64_t)pl.T + 1;
  z.chunk_tile = pl.max_chunks;
  z.record_words = (samples > 0 ? samples : 1) * (uint64_t)(dim + 2);
  z.scratch_floats = (uint64_t)pl.max_chunks * pl.rcells * pl.C;
  auto al = [](uint64_t b) { return (b + 255) & ~(uint64_t)255; };
  z.total_bytes = al(z.counts * 4) + al(z.bin_start * 4) + al(z.chunk_off * 4) +
                  al(z.chunk_tile * 4) + al(z.record_words * 4) + al(z.scratch_floats * 4);
  return z;
}

hipError_t run_bwd(const BwdPlan& pl, const BwdBuffers& bf, int dim, int vdt, int cdt,
                   int vec_bytes, hipStream_t s) {
  BwdFn fn = get_bwd(dim, vdt, cdt, vec_bytes);
  if (!fn) return hipErrorInvalidValue;
  return fn(pl, bf, s);
}

}  // namespace msda
