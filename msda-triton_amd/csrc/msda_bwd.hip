// msda_bwd.hip — gfx950 backward of multi-scale deformable attention without global
// floating-point atomics.
//
// Replaces the reference's _bwd_kernel_2d (src/msda_triton/triton/msda_2d.py:263-510) and
// 3D _bwd_kernel (src/msda_triton/triton/msda_3d.py:291-653), which scatter grad_value
// with one global atomic per (sample, corner, channel). On MI355X global fp32 atomics
// sustain only tens of G element-adds/s, so this backward accumulates grad_value in key
// order instead:
//
//  1. bin (count): every sample is assigned to the spatial tiles of its level that own
//     its valid corner cells (1 to 2^dim tiles). Each workgroup covers the units of one
//     (batch, head-group), histograms its records per tile in LDS, and writes the
//     histogram as one column of a per-(tile, workgroup) count matrix.
//  2. exclusive scan of the count matrix (tile-major): every (tile, workgroup) pair gets
//     a disjoint, contiguous record range; no global atomics are involved.
//  3. bin (fill): the same traversal writes each record (q*P + p, plus a "primary" bit
//     for the tile of the sample's lowest valid corner) at its range base + LDS rank.
//  4. chunk table: each tile's records are cut into chunks of at most R records.
//  5. tile kernel: one workgroup per chunk stages the tile's value rows (the tile plus a
//     one-cell halo on the high side) in LDS, and for every record accumulates
//     attn * w_corner * grad_out into the LDS accumulator of the owned corners (LDS
//     atomics). For primary records it also forms <grad_out, value_corner> from the staged
//     rows and writes grad_attention_weights and grad_sampling_locations with plain
//     stores. A tile with one chunk writes its grad_value cells directly in the value
//     dtype; a tile with several chunks writes fp32 partials.
//  6. reduce: sums the partials of multi-chunk tiles and writes their grad_value cells.
//
// Every grad_value element is written exactly once with a plain store, so no clearing
// pass is needed and 16-bit values need no fp32 staging copy.
#include "msda_internal.h"
#include "msda_sample.h"

namespace msda {

namespace {

constexpr int kScanItems = 8;
constexpr int kScanTile = kBlock * kScanItems;

// ------------------------------------------------------------------ exclusive scan
__device__ inline uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t t = __shfl_up(v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

// Exclusive scan of one value per thread across the workgroup; *total gets the sum.
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* s_w, uint32_t* total) {
  const uint32_t inc = wave_incl_scan(v);
  const int w = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  if (lane == kWave - 1) s_w[w] = inc;
  __syncthreads();
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kBlock / kWave; ++i) {
    const uint32_t x = s_w[i];
    if (i < w) pre += x;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return pre + inc - v;
}

template <int NT>
__device__ inline uint32_t block_excl_scan_n(uint32_t v, uint32_t* s_w, uint32_t* total) {
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

__global__ __launch_bounds__(kBlock) void scan_reduce_kernel(const uint32_t* a, uint32_t n,
                                                             uint32_t* sums) {
  __shared__ uint32_t s_w[kBlock / kWave];
  const uint32_t base = blockIdx.x * kScanTile;
  uint32_t v = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const uint32_t k = base + i * kBlock + threadIdx.x;
    if (k < n) v += a[k];
  }
  uint32_t tot;
  block_excl_scan(v, s_w, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

// Single workgroup: exclusive scan of nb block sums in place; a[n] = grand total.
__global__ __launch_bounds__(kBlock) void scan_sums_kernel(uint32_t* sums, uint32_t nb,
                                                           uint32_t* a, uint32_t n) {
  __shared__ uint32_t s_w[kBlock / kWave];
  uint32_t carry = 0;
  for (uint32_t base = 0; base < nb; base += kBlock) {
    const uint32_t k = base + threadIdx.x;
    const uint32_t v = k < nb ? sums[k] : 0u;
    uint32_t tot;
    const uint32_t ex = block_excl_scan(v, s_w, &tot);
    if (k < nb) sums[k] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) a[n] = carry;
}

__global__ __launch_bounds__(kBlock) void scan_apply_kernel(uint32_t* a, uint32_t n,
                                                            const uint32_t* sums) {
  __shared__ uint32_t s_w[kBlock / kWave];
  const uint32_t base = blockIdx.x * kScanTile + threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t run = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    v[i] = base + i < n ? a[base + i] : 0u;
    run += v[i];
  }
  uint32_t tot;
  uint32_t pre = block_excl_scan(run, s_w, &tot) + sums[blockIdx.x];
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    if (base + i < n) a[base + i] = pre;
    pre += v[i];
  }
}

hipError_t scan_inplace(uint32_t* a, uint32_t n, uint32_t* sums, hipStream_t s) {
  const uint32_t nb = (n + kScanTile - 1) / kScanTile;
  if (nb > 0) {
    hipLaunchKernelGGL(scan_reduce_kernel, dim3(nb), dim3(kBlock), 0, s, a, n, sums);
  }
  hipLaunchKernelGGL(scan_sums_kernel, dim3(1), dim3(kBlock), 0, s, sums, nb, a, n);
  if (nb > 0) {
    hipLaunchKernelGGL(scan_apply_kernel, dim3(nb), dim3(kBlock), 0, s, a, n, sums);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ tiles of a sample
// Tiles (along one axis) owning the valid corners of a sample: first tile t0 and count
// n in {0, 1, 2}; the corners are adjacent, so a second tile is always t0 + 1.
struct AxisTiles {
  int t0, n;
};

__device__ inline AxisTiles axis_tiles(const Axis& a, int T) {
  AxisTiles r;
  if (a.v0) {
    r.t0 = a.i0 / T;
    r.n = (a.v1 && (a.i0 + 1) / T != r.t0) ? 2 : 1;
  } else if (a.v1) {
    r.t0 = (a.i0 + 1) / T;
    r.n = 1;
  } else {
    r.t0 = 0;
    r.n = 0;
  }
  return r;
}

struct TileCoord {
  uint32_t b, h;
  int l, X0, Y0, Z0;
};

__device__ inline TileCoord decode_tile(const BwdPlan& pl, uint32_t t) {
  TileCoord tc;
  const uint32_t g = t / (uint32_t)pl.bins, bin = t - g * (uint32_t)pl.bins;
  const uint32_t hsub = bin / (uint32_t)pl.tiles_per_bh;
  const int tib = (int)(bin - hsub * (uint32_t)pl.tiles_per_bh);
  const uint32_t gph = (uint32_t)pl.H >> pl.hg_log2;
  tc.b = g / gph;
  tc.h = ((g - tc.b * gph) << pl.hg_log2) | hsub;
  int l = 0;
  while (l + 1 < pl.L && pl.lv[l + 1].tile_off <= tib) ++l;
  tc.l = l;
  const BwdLevel& lv = pl.lv[l];
  const int lt = tib - lv.tile_off;
  tc.X0 = (lt % lv.ntx) * pl.TX;
  tc.Y0 = ((lt / lv.ntx) % lv.nty) * pl.TY;
  tc.Z0 = (lt / (lv.ntx * lv.nty)) * pl.TZ;
  return tc;
}

// ------------------------------------------------------------------ 1, 3: binning
template <int DIM, typename EC, bool FILL>
__global__ __launch_bounds__(kBlock) void bwd_bin_kernel(const BwdPlan pl, const BwdBuffers bf) {
  typedef typename EC::T TC;
  extern __shared__ uint32_t s_hist[];  // [bins] counters, then [bins] record bases (fill)
  uint32_t* s_base = s_hist + pl.bins;
  const uint32_t g = blockIdx.x / (uint32_t)pl.wgpg;
  const uint32_t w = blockIdx.x - g * (uint32_t)pl.wgpg;
  for (int i = threadIdx.x; i < pl.bins; i += kBlock) {
    s_hist[i] = 0;
    if (FILL) s_base[i] = bf.counts[((size_t)g * pl.bins + i) * pl.wgpg + w];
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
    for (int l = 0; l < pl.L; ++l) {
      const BwdLevel& lv = pl.lv[l];
      const Level lvl = {lv.start, lv.W, lv.H, lv.D};
      for (int p = 0; p < pl.P; ++p) {
        const int s = l * pl.P + p;
        const Sample<DIM> sm = make_sample<DIM>(locp + s * DIM, lvl, pl.clamp, pl.lo_g, pl.hi_g);
        const AxisTiles tx = axis_tiles(sm.ax, pl.TX);
        const AxisTiles ty = axis_tiles(sm.ay, pl.TY);
        AxisTiles tz = {0, 1};
        if constexpr (DIM == 3) tz = axis_tiles(sm.az, pl.TZ);
        if (tx.n == 0 || ty.n == 0 || tz.n == 0) {
          // no corner inside the level: the sample's gradients are zero
          if (!FILL) {
            TC* gl = static_cast<TC*>(bf.grad_loc) + (bqh * LP + s) * DIM;
#pragma unroll
            for (int d = 0; d < DIM; ++d) gl[d] = (TC)0.0f;
            static_cast<TC*>(bf.grad_attn)[bqh * LP + s] = (TC)0.0f;
          }
          continue;
        }
        for (int iz = 0; iz < tz.n; ++iz)
          for (int iy = 0; iy < ty.n; ++iy)
            for (int ix = 0; ix < tx.n; ++ix) {
              const int tib = lv.tile_off + ((tz.t0 + iz) * lv.nty + ty.t0 + iy) * lv.ntx + tx.t0 + ix;
              const uint32_t bin = hsub * (uint32_t)pl.tiles_per_bh + (uint32_t)tib;
              const uint32_t r = atomicAdd(&s_hist[bin], 1u);
              if (FILL) {
                const uint32_t prim = (ix | iy | iz) == 0 ? 0x80000000u : 0u;
                bf.records[s_base[bin] + r] = (q * (uint32_t)pl.P + (uint32_t)p) | prim;
              }
            }
      }
    }
  }
  if (!FILL) {
    __syncthreads();
    for (int i = threadIdx.x; i < pl.bins; i += kBlock)
      bf.counts[((size_t)g * pl.bins + i) * pl.wgpg + w] = s_hist[i];
  }
}

// ------------------------------------------------------------------ 4: chunk table
__global__ __launch_bounds__(kBlock) void tile_nch_kernel(const BwdPlan pl, const BwdBuffers bf) {
  const uint32_t t = blockIdx.x * kBlock + threadIdx.x;
  if (t >= pl.T) return;
  const uint32_t n = bf.counts[(size_t)(t + 1) * pl.wgpg] - bf.counts[(size_t)t * pl.wgpg];
  const uint32_t nch = (n + pl.R - 1) / pl.R;
  bf.tile_nch[t] = nch > 0 ? nch : 1u;  // an empty tile still gets one chunk (writes zeros)
}

__global__ __launch_bounds__(kBlock) void chunk_table_kernel(const BwdPlan pl, const BwdBuffers bf) {
  const uint32_t t = blockIdx.x * kBlock + threadIdx.x;
  if (t >= pl.T) return;
  const uint32_t off = bf.tile_nch[t], end = bf.tile_nch[t + 1];
  for (uint32_t c = off; c < end; ++c) bf.chunk_tile[c] = t;
}

// ------------------------------------------------------------------ 5: tile kernel
// One workgroup (kTileThreads threads) per chunk of a tile's records. LDS holds the staged
// value region, and per sub-batch of up to S records: each record's grad_out row, the
// (weight, record) entries of the owned corners sorted by cell, and per-cell counters.
// Per sub-batch:
//   A. record pass (2^lpu_log2 lanes per record): stage the grad_out row; for primary
//      records form <grad_out, value_corner> from the staged value rows and store
//      grad_attention_weights / grad_sampling_locations; count owned corners per cell.
//   B. exclusive scan of the per-cell counts.
//   C. entry pass (one thread per record): place (attn * w_corner, record) entries of the
//      owned corners at their cell's offset + rank.
//   D. owner pass: the thread owning (cell, channel chunk) sums attn*w*grad_out over its
//      cell's entries in fp32 registers.
// Only 32-bit integer LDS atomics are used (LDS float atomics are far slower on gfx950).
template <int DIM, typename EV, typename EC, int VEC>
__global__ __launch_bounds__(kTileThreads) void bwd_tile_kernel(const BwdPlan pl,
                                                                const BwdBuffers bf) {
  constexpr int VB = VEC * EV::kBytes;
  constexpr int NC = 1 << DIM;
  constexpr int MI = kTileMaxItems;  // owner items per thread
  typedef typename EC::T TC;
  typedef typename EV::T TV;
  extern __shared__ __attribute__((aligned(16))) char s_mem[];

  const uint32_t c = blockIdx.x;
  if (c >= bf.tile_nch[pl.T]) return;  // beyond the real chunk count: the whole block exits
  const uint32_t t = bf.chunk_tile[c];
  const uint32_t off = bf.tile_nch[t];
  const uint32_t nch = bf.tile_nch[t + 1] - off;
  const uint32_t rbeg = bf.counts[(size_t)t * pl.wgpg];
  const uint32_t rend = bf.counts[(size_t)(t + 1) * pl.wgpg];
  const uint32_t beg = rbeg + (c - off) * pl.R;
  const uint32_t end = min(rend, beg + pl.R);
  const TileCoord tc = decode_tile(pl, t);
  const BwdLevel lv = pl.lv[tc.l];
  const Level lvl = {lv.start, lv.W, lv.H, lv.D};

  char* s_val = s_mem;
  char* s_g = s_mem + pl.lds_val_bytes;                                    // [S][C] raw rows
  uint2* s_ent = reinterpret_cast<uint2*>(s_g + pl.lds_g_bytes);           // [S * NC]
  uint32_t* s_cnt = reinterpret_cast<uint32_t*>(s_ent + (size_t)pl.S * NC);  // [cells + 1]
  uint32_t* s_cur = s_cnt + pl.cells + 1;                                  // [cells]
  uint32_t* s_w = s_cur + pl.cells;                                        // [waves]
  const int ncell_r = pl.RX * pl.RY * pl.RZ;
  const int ncell_o = pl.cells;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(bf.value, pl.value_bytes);
  const uint32_t rs = (uint32_t)pl.H * (uint32_t)pl.C * EV::kBytes;
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
    for (int i = threadIdx.x; i <= ncell_o; i += kTileThreads) s_cnt[i] = 0u;
    __syncthreads();  // value region staged (first sub-batch); counters cleared

    // A. record pass
    for (uint32_t r = grp; r < nrec; r += groups) {
      const uint32_t rec = bf.records[sb + r];
      const bool primary = (rec >> 31) != 0;
      const uint32_t qp = rec & 0x7fffffffu;
      const uint32_t q = fdiv(qp, pl.div_p), p = qp - q * (uint32_t)pl.P;
      const size_t bqh = ((size_t)tc.b * pl.Q + q) * pl.H + tc.h;
      const size_t si = bqh * LP + (size_t)tc.l * pl.P + p;
      const Sample<DIM> sm =
          make_sample<DIM>(static_cast<const TC*>(bf.loc) + si * DIM, lvl, pl.clamp, pl.lo_g, pl.hi_g);
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
      // count the owned corners, one lane per corner
      for (int cc = (int)lane; cc < NC; cc += (int)lanes) {
        const int ox = sm.ax.i0 + (cc & 1) - tc.X0, oy = sm.ay.i0 + ((cc >> 1) & 1) - tc.Y0;
        const int oz = DIM == 3 ? sm.az.i0 + ((cc >> 2) & 1) - tc.Z0 : 0;
        if (corner_valid<DIM>(cc, sm) && (unsigned)ox < (unsigned)pl.TX &&
            (unsigned)oy < (unsigned)pl.TY && (unsigned)oz < (unsigned)pl.TZ)
          atomicAdd(&s_cnt[(oz * pl.TY + oy) * pl.TX + ox], 1u);
      }
      if (primary) {
        float dot[NC];
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          const int ox = sm.ax.i0 + (cc & 1) - tc.X0, oy = sm.ay.i0 + ((cc >> 1) & 1) - tc.Y0;
          const int oz = DIM == 3 ? sm.az.i0 + ((cc >> 2) & 1) - tc.Z0 : 0;
          dot[cc] = 0.0f;
          if (act && corner_valid<DIM>(cc, sm) && (unsigned)ox < (unsigned)pl.RX &&
              (unsigned)oy < (unsigned)pl.RY && (unsigned)oz < (unsigned)pl.RZ) {
            const RawVec<VB> rw = *reinterpret_cast<const RawVec<VB>*>(
                s_val + ((oz * pl.RY + oy) * pl.RX + ox) * pl.val_row_bytes + lane * VB);
            float v[VEC];
            widen<EV, VEC>(rw, v);
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
          const float a = (float)static_cast<const TC*>(bf.attn)[si];
          static_cast<TC*>(bf.grad_attn)[si] = (TC)s_attn;
          TC* gl = static_cast<TC*>(bf.grad_loc) + si * DIM;
          gl[0] = (TC)(sm.ax.pass ? (a * s_x) * (float)lv.W : 0.0f);
          gl[1] = (TC)(sm.ay.pass ? (a * s_y) * (float)lv.H : 0.0f);
          if constexpr (DIM == 3) gl[2] = (TC)(sm.az.pass ? (a * s_z) * (float)lv.D : 0.0f);
        }
      }
    }
    __syncthreads();

    // B. exclusive scan of the per-cell counts (cells <= kTileThreads)
    {
      const uint32_t v = (int)threadIdx.x < ncell_o ? s_cnt[threadIdx.x] : 0u;
      uint32_t tot;
      const uint32_t ex = block_excl_scan_n<kTileThreads>(v, s_w, &tot);
      if ((int)threadIdx.x < ncell_o) {
        s_cnt[threadIdx.x] = ex;
        s_cur[threadIdx.x] = 0u;
      }
      if (threadIdx.x == 0) s_cnt[ncell_o] = tot;
    }
    __syncthreads();

    // C. entry pass: one thread per record
    for (uint32_t r = threadIdx.x; r < nrec; r += kTileThreads) {
      const uint32_t qp = bf.records[sb + r] & 0x7fffffffu;
      const uint32_t q = fdiv(qp, pl.div_p), p = qp - q * (uint32_t)pl.P;
      const size_t si = (((size_t)tc.b * pl.Q + q) * pl.H + tc.h) * LP + (size_t)tc.l * pl.P + p;
      const Sample<DIM> sm =
          make_sample<DIM>(static_cast<const TC*>(bf.loc) + si * DIM, lvl, pl.clamp, pl.lo_g, pl.hi_g);
      const float a = (float)static_cast<const TC*>(bf.attn)[si];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const int ox = sm.ax.i0 + (cc & 1) - tc.X0, oy = sm.ay.i0 + ((cc >> 1) & 1) - tc.Y0;
        const int oz = DIM == 3 ? sm.az.i0 + ((cc >> 2) & 1) - tc.Z0 : 0;
        if (corner_valid<DIM>(cc, sm) && (unsigned)ox < (unsigned)pl.TX &&
            (unsigned)oy < (unsigned)pl.TY && (unsigned)oz < (unsigned)pl.TZ) {
          const int cell = (oz * pl.TY + oy) * pl.TX + ox;
          const uint32_t pos = s_cnt[cell] + atomicAdd(&s_cur[cell], 1u);
          const float cw = corner_weight<DIM>(cc, sm) * a;
          s_ent[pos] = make_uint2(__builtin_bit_cast(uint32_t, cw), r);
        }
      }
    }
    __syncthreads();

    // D. owner pass: fp32 register accumulation per (cell, channel chunk)
#pragma unroll
    for (int m = 0; m < MI; ++m) {
      const int it = (int)threadIdx.x + m * kTileThreads;
      if (it < ncell_o * pl.nvec) {
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

  // write the owned cells: directly in the value dtype for a single-chunk tile, else as an
  // fp32 partial for the reduce kernel
#pragma unroll
  for (int m = 0; m < MI; ++m) {
    const int it = (int)threadIdx.x + m * kTileThreads;
    if (it >= ncell_o * pl.nvec) continue;
    const int cell = it / pl.nvec, ch = it - cell * pl.nvec;
    if (nch == 1) {
      const int x = tc.X0 + cell % pl.TX, y = tc.Y0 + (cell / pl.TX) % pl.TY;
      const int z = tc.Z0 + cell / (pl.TX * pl.TY);
      if (x < lv.W && y < lv.H && z < lv.D) {
        const uint32_t row = (uint32_t)lv.start + ((uint32_t)z * lv.H + y) * lv.W + x;
        store_vec<EV, VEC>(static_cast<TV*>(bf.grad_value) +
                               (((size_t)tc.b * pl.K + row) * pl.H + tc.h) * pl.C + ch * VEC,
                           acc[m]);
      }
    } else {
      float* dst = bf.scratch + ((size_t)c * ncell_o + cell) * pl.C + ch * VEC;
#pragma unroll
      for (int k = 0; k < VEC; ++k) dst[k] = acc[m][k];
    }
  }
}

// ------------------------------------------------------------------ 6: reduce
template <typename EV, int VEC>
__global__ __launch_bounds__(kBlock) void bwd_reduce_kernel(const BwdPlan pl, const BwdBuffers bf) {
  typedef typename EV::T TV;
  const uint32_t t = blockIdx.x;
  const uint32_t off = bf.tile_nch[t];
  const uint32_t nch = bf.tile_nch[t + 1] - off;
  if (nch <= 1) return;
  const TileCoord tc = decode_tile(pl, t);
  const BwdLevel lv = pl.lv[tc.l];
  const int ncell_o = pl.TX * pl.TY * pl.TZ;
  TV* gv = static_cast<TV*>(bf.grad_value);
  for (int i = threadIdx.x; i < ncell_o * pl.nvec; i += kBlock) {
    const int cell = i / pl.nvec, ch = i - cell * pl.nvec;
    const int x = tc.X0 + cell % pl.TX, y = tc.Y0 + (cell / pl.TX) % pl.TY;
    const int z = tc.Z0 + cell / (pl.TX * pl.TY);
    if (x >= lv.W || y >= lv.H || z >= lv.D) continue;
    float o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = 0.0f;
    for (uint32_t j = 0; j < nch; ++j) {
      const float* src = bf.scratch + ((size_t)(off + j) * ncell_o + cell) * pl.C + ch * VEC;
#pragma unroll
      for (int k = 0; k < VEC; ++k) o[k] += src[k];
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
  const uint32_t ncount = pl.T * (uint32_t)pl.wgpg;
  hipError_t e = scan_inplace(bf.counts, ncount, bf.scan_tmp, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_bin_kernel<DIM, EC, true>), dim3(nbin_wg), dim3(kBlock), 2 * hist_bytes,
                     s, pl, bf);
  if (pl.T == 0) return hipGetLastError();  // no cell in any level: grad_value is empty
  const dim3 tgrid((pl.T + kBlock - 1) / kBlock);
  hipLaunchKernelGGL(tile_nch_kernel, tgrid, dim3(kBlock), 0, s, pl, bf);
  e = scan_inplace(bf.tile_nch, pl.T, bf.scan_tmp, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(chunk_table_kernel, tgrid, dim3(kBlock), 0, s, pl, bf);
  hipLaunchKernelGGL((bwd_tile_kernel<DIM, EV, EC, VEC>), dim3(pl.max_chunks),
                     dim3(kTileThreads), pl.lds_bytes, s, pl, bf);
  hipLaunchKernelGGL((bwd_reduce_kernel<EV, VEC>), dim3(pl.T), dim3(kBlock), 0, s, pl, bf);
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

BwdSizes bwd_sizes(const BwdPlan& pl, uint64_t records) {
  BwdSizes z;
  z.counts = (uint64_t)pl.T * pl.wgpg + 1;
  const uint64_t nscan = z.counts > (uint64_t)pl.T + 1 ? z.counts : (uint64_t)pl.T + 1;
  z.scan_tmp = (nscan + kScanTile - 1) / kScanTile + 1;
  z.records = records > 0 ? records : 1;
  z.tile_nch = (uint64_t)pl.T + 1;
  z.chunk_tile = pl.max_chunks;
  z.scratch_floats = (uint64_t)pl.max_chunks * pl.TX * pl.TY * pl.TZ * pl.C;
  auto al = [](uint64_t b) { return (b + 255) & ~(uint64_t)255; };
  z.total_bytes = al(z.counts * 4) + al(z.scan_tmp * 4) + al(z.records * 4) + al(z.tile_nch * 4) +
                  al(z.chunk_tile * 4) + al(z.scratch_floats * 4);
  return z;
}

hipError_t run_bwd(const BwdPlan& pl, const BwdBuffers& bf, int dim, int vdt, int cdt,
                   int vec_bytes, hipStream_t s) {
  BwdFn fn = get_bwd(dim, vdt, cdt, vec_bytes);
  if (!fn) return hipErrorInvalidValue;
  return fn(pl, bf, s);
}

}  // namespace msda
