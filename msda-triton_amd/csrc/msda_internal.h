// msda_internal.h — host <-> kernel parameter blocks and launcher declarations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "msda_device.h"

namespace msda {

constexpr int kMaxLevels = 64;
// threads of the backward tile kernel: 2D 256 (four workgroups per CU, 16x8-cell tiles),
// 3D 512 (two workgroups per CU: smaller workgroups would shrink the 3D tiles to 4x4x4 and
// double the bins and the fill's work)
template <int DIM>
constexpr int kTileThreads = DIM == 2 ? 256 : 512;
// channels per owner item of the tile kernel for VEC channels per value load and eb bytes
// per staged element: 16 staged bytes, so the lanes of one cell read a staged row in one
// conflict-free pass (four fp32 or eight 16-bit channels)
constexpr int tile_owner_vec(int vec, int eb) { return vec < 16 / eb ? vec : 16 / eb; }
// (region cell, channel chunk) owner items per tile thread: 20-24 fp32 accumulators
constexpr int tile_max_items(int ov) { return ov >= 8 ? 3 : 5; }
// words per backward record: 16-bit coordinates 3 (id | flags, then the raw 16-bit
// location and weight two to a word), fp32 coordinates dim + 2 (id | flags, the pixel
// coordinates and the weight)
constexpr int record_words(int dim, int coord_bytes) { return coord_bytes == 2 ? 3 : dim + 2; }
constexpr int kTileWavesPerSimd = 4;  // tile-kernel occupancy target (128 VGPRs)
constexpr int kFillStage = 2048;      // records staged in LDS per fill round
constexpr int kGradThreads = 256;     // threads of the backward count, fill and atomic kernels
// units (b, q, h) of a count / fill workgroup: kGradRounds unit groups of 2^lpu_log2 lanes per
// thread. 3D launches that keep at least kGradWgsPerCu workgroups per CU at twice as many
// rounds use 2 * kGradRounds (C5 fill 113 -> 110 us)
constexpr int kGradRounds = 4;
constexpr int kGradWgsPerCu = 2;
// threads of the staged forward kernel: 12 waves per CU leave each lane 168 VGPRs, so
// neither variant spills (at 1024 threads, 128 VGPRs, the plain kernel spilled 20-64 bytes
// per lane and the fused one 70-116, and both ran slower; 512 and 896 threads were slower)
constexpr int kFwdStageThreads = 768;
constexpr uint32_t kFwdStageLds = 156 * 1024;     // its dynamic LDS: one workgroup per CU
constexpr uint32_t kFwdStageMinQueries = 512;     // queries per workgroup that pay for staging
// coordinate blocks a forward lane holds (2D: 4-sample blocks, 3D: 2-sample blocks)
template <int DIM>
constexpr int kFwdCoordSlots = DIM == 2 ? 2 : 4;

// Forward parameters for one launch over a contiguous range of batches. Pointers are
// already offset to the first batch of the range; all in-kernel offsets are 32-bit.
struct Params {
  const void* value;       // (Bc, K, H, C) value_dtype
  const void* loc;         // (Bc, Q, H, L, P, dim) coord_dtype
  const void* attn;        // (Bc, Q, H, L, P) coord_dtype
  void* out;               // (Bc, Q, H*C) value_dtype
  const int32_t* shapes;   // (L, dim) device
  const int32_t* starts;   // (L,) device
  uint32_t value_bytes;    // bytes of value in this launch (< 2^31)
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
  uint32_t xcds;           // XCDs of the device (workgroups are dealt to them round-robin)
  int32_t coords_aligned;  // loc and attn are 16-byte aligned: per-level block loads allowed
  // staged path: one workgroup per (batch, head, query range) keeps the smallest levels of
  // its (batch, head) value slice in LDS
  uint32_t splits;         // workgroups per (batch, head)
  uint32_t qper;           // queries per workgroup
  uint32_t stage_bytes;    // LDS bytes for staged rows
  // head-major copy of value, (Bc, H, K, C), or nullptr: rows are then read from it with
  // the rows of one head contiguous
  const void* value_h;
  // fused producer launches: loc holds the sampling offsets (Bc, Q, H, L, P, dim) and attn
  // the attention logits (Bc, Q, H, L, P), both coord_dtype; ref the fp32 reference points
  // (Bc, Q, L, dim). The kernel forms loc = ref + off / (W, H[, D]) and attn = softmax over
  // (L, P) in fp32.
  const float* ref;
};

using LaunchFn = hipError_t (*)(const Params&, hipStream_t);

// Copy value (B, K, H, row_bytes) into head-major order (B, H, K, row_bytes), vec_bytes
// (16, 8, 4 or 2, dividing row_bytes and the pointers' alignment) per thread and load.
hipError_t launch_head_major(const void* src, void* dst, uint32_t B, uint32_t K, uint32_t H,
                             uint32_t row_bytes, int vec_bytes, hipStream_t s);

// Forward launcher for (dim, value dtype, coord dtype, bytes per lane load), or nullptr.
// `staged` selects the kernel that serves small levels from LDS (Params.splits/qper set);
// `fused` the kernels that form locations and weights from offsets and logits (Params.ref).
LaunchFn get_fwd_launcher(int dim, int vdt, int cdt, int vec_bytes, bool staged, bool fused);

// ---------------------------------------------------------------------------------------
// Backward. grad_value is accumulated in key order. Every sample with a valid corner is
// binned to the spatial tile of its level that owns its lowest corner; the tile's value
// region (the tile plus a one-cell halo on the high side of each axis) then holds all of
// the sample's corners. One workgroup per chunk of a tile's records stages that region
// in LDS, computes grad_sampling_locations and grad_attention_weights of its samples
// from the staged rows, and accumulates grad_value for the region in fp32 registers of
// the cell owners (records are sorted by cell in LDS with integer LDS atomics). Interior
// cells of a tile processed by one chunk are written directly; edge cells, halo cells and
// split tiles go through fp32 partials that a fold kernel sums, in a fixed order, into
// the cells' final values.
constexpr uint32_t kRecIdBits = 27;                     // record id = q * P + p
constexpr uint32_t kRecIdMask = (1u << kRecIdBits) - 1u;
constexpr uint32_t kRecPassX = 1u << 27;                // grid clamp inactive on x / y / z
constexpr uint32_t kRecPassY = 1u << 28;
constexpr uint32_t kRecPassZ = 1u << 29;

struct BwdLevel {
  int32_t start, W, H, D;      // first row in K and extents (D = 1 in 2D)
  int32_t ntx, nty, ntz;       // tiles along x, y, z
  int32_t tile_off;            // index of the level's first tile within a (b, h); the
                               // coarsest level comes first so its long chunks start early
  int32_t ntiles;              // ntx * nty * ntz
  uint32_t base;               // start * rs: byte offset of the level's first row in a (b, h) slice
  int32_t sy, sz;              // byte strides along y and z (W * rs, H * W * rs); x is rs
};

// Level geometry of one backward launch: what depends on the level shapes. It lives in
// the workspace and the kernels read it through a constant-address-space pointer, so a
// wave-uniform field is one scalar load, as a kernel argument would be. Host-resident
// shapes: computed on the host and passed to the first kernel, which stores it.
// Device-resident shapes: computed by bwd_geom_kernel from the shapes on the device, so the
// host never reads them (no device-to-host copy, no synchronisation; the launch sequence
// can be graph-captured).
struct BwdGeom {
  BwdLevel lv[kMaxLevels];
  int32_t tiles_per_bh;        // tiles of all levels of one (b, h)
  int32_t bins;                // tiles_per_bh * HG; bin = tile_in_bh * HG + head_in_group
  uint32_t T;                  // groups * bins: tiles of this launch
  int32_t mul24;               // every row stride and corner index fits 24-bit multiplies
  int32_t atomic;              // grad_value goes through fp32 atomics into BwdBuffers::sums
                               // (levels beyond the binning capacity, or invalid shapes)
  int32_t invalid;             // device shapes disagree with K (or overflow 32-bit offsets):
                               // every gradient is filled with NaN
  int32_t pad[2];
};

// Inputs of make_geom besides the shapes (all known on the host without the shapes).
struct GeomArgs {
  int32_t dim, L, H, C, s;     // s = bytes per value element
  int32_t head_major;          // rows of one head contiguous (head-major value copy)
  int32_t hg_log2, groups;
  int32_t TX, TY, TZ;
  int32_t bins_cap;            // bins the launch was sized for; more -> atomic path
  int32_t static_atomic;       // the host already chose the atomic path
  int64_t K;
};

// Tiles along one axis of extent n for tiles of t cells.
__host__ __device__ inline int32_t tiles_along(int32_t n, int32_t t) { return (n + t - 1) / t; }

// The level geometry of a launch from the (L, dim) int32 shapes (rows (H, W) or (D, H, W)).
// Shared by the host planner and bwd_geom_kernel so both paths compute the same table.
__host__ __device__ inline void make_geom(const GeomArgs& a, const int32_t* hs, BwdGeom* g) {
  int64_t total = 0;
  bool bad = false;
  const uint64_t rsb = (uint64_t)(a.head_major ? 1 : a.H) * a.C * a.s;  // bytes between rows of K
  bool mul24 = rsb < (1u << 23);
  int32_t tiles = 0;
  for (int l = 0; l < a.L; ++l) {
    BwdLevel& lv = g->lv[l];
    const int32_t d0 = hs[l * a.dim], d1 = hs[l * a.dim + 1];
    const int32_t d2 = a.dim == 3 ? hs[l * a.dim + 2] : 1;
    lv.D = a.dim == 3 ? d0 : 1;
    lv.H = a.dim == 3 ? d1 : d0;
    lv.W = a.dim == 3 ? d2 : d1;
    if (lv.D < 0 || lv.H < 0 || lv.W < 0) bad = true;
    lv.start = (int32_t)total;
    if (!bad) total += (int64_t)lv.D * lv.H * lv.W;
    if (total > 0x7FFFFFFFll) bad = true;
  }
  if (total != a.K) bad = true;
  for (int l = a.L - 1; l >= 0; --l) {  // coarsest level first: its chunks are the longest
    BwdLevel& lv = g->lv[l];
    if (bad) {
      lv = BwdLevel{};
      continue;
    }
    lv.base = (uint32_t)((uint64_t)lv.start * rsb);
    lv.sy = (int32_t)((uint64_t)lv.W * rsb);
    lv.sz = (int32_t)((uint64_t)lv.W * lv.H * rsb);
    // largest stride used (y in 2D, z in 3D) and largest corner index must fit 24 bits
    const uint64_t top = (uint64_t)lv.W * (a.dim == 3 ? (uint64_t)lv.H : 1u) * rsb;
    const int64_t ext = (lv.W > lv.H ? (lv.W > lv.D ? lv.W : lv.D) : (lv.H > lv.D ? lv.H : lv.D)) + 2;
    if (top >= (1u << 23) || ext >= (1 << 23)) mul24 = false;
    lv.ntx = tiles_along(lv.W, a.TX);
    lv.nty = tiles_along(lv.H, a.TY);
    lv.ntz = tiles_along(lv.D, a.TZ);
    lv.tile_off = tiles;
    const int64_t nt = a.static_atomic ? 0 : (int64_t)lv.ntx * lv.nty * lv.ntz;
    lv.ntiles = (int32_t)(nt < 0x40000000 ? nt : 0x40000000);
    tiles = tiles + lv.ntiles < 0x40000000 ? tiles + lv.ntiles : 0x40000000;
  }
  const int64_t bins = (int64_t)tiles << a.hg_log2;
  const bool over = bins > a.bins_cap;
  g->tiles_per_bh = over || bad ? 0 : tiles;
  g->bins = over || bad ? 0 : (int32_t)bins;
  g->T = (uint32_t)a.groups * (uint32_t)g->bins;
  g->mul24 = mul24 && !bad ? 1 : 0;
  g->atomic = (a.static_atomic || over || bad) ? 1 : 0;
  g->invalid = bad ? 1 : 0;
  g->pad[0] = g->pad[1] = 0;
}

struct BwdPlan {
  int32_t L, P, C, H, K;
  uint32_t Q;
  FastDiv div_p;               // divisor P (record id -> q, p)
  FastDiv div_lp;              // divisor L * P (sample index -> unit, sample)
  int32_t TX, TY, TZ;          // owned cells per tile, powers of two (TZ = 1 in 2D)
  int32_t tx_log2, ty_log2, tz_log2;
  FastDiv div_nvec;            // divisor nvec (value-load chunks per row)
  int32_t onv;                 // owner chunks per row in the tile kernel: C / tile_owner_vec(VEC, s)
  FastDiv div_onv;             // divisor onv (owner item -> cell, chunk)
  FastDiv div_tx, div_txy;     // divisors TX and TX * TY (owned cell -> lx, ly, lz)
  int32_t RX, RY, RZ;          // region: tile + 1 along each axis (RZ = 1 in 2D)
  int32_t cells;               // owned cells per tile: TX * TY * TZ
  int32_t rcells;              // region cells per tile: RX * RY * RZ
  int32_t hg_log2;
  int32_t groups;              // (batches in launch) * H / HG
  int32_t upw;                 // units (b, q, h) per bin workgroup: rounds * kGradThreads / lanes per unit
  int32_t wgpg;                // bin workgroups per group: ceil(Q * HG / upw)
  int32_t bins_cap;            // bins the LDS histograms and the count matrix are sized for
  uint32_t T_cap;              // groups * bins_cap: tiles the tables and grids are sized for
  uint32_t R;                  // records per chunk (multiple of S)
  uint32_t S;                  // records per LDS sub-batch of the tile kernel (<= kTileThreads<DIM>)
  int32_t lpu_log2, nvec;
  int32_t clamp;
  int32_t coords_aligned;      // loc and attn are 16-byte aligned: per-batch block loads allowed
  int32_t head_major;          // value is the caller's head-major (B, H, K, C) copy
                               // (MSDA_FLAG_VALUE_HEAD_MAJOR): the tile kernel's region rows,
                               // the atomic path's gathers and its fp32 sums follow that layout
  int32_t static_atomic;       // the host chose the atomic path (levels beyond the LDS binning,
                               // or sample ids beyond a record): grad_value is scattered with
                               // fp32 atomics into BwdBuffers::sums, then rounded into grad_value
  int32_t fallback;            // device shapes: the binned and the atomic kernels are both
                               // launched and each exits unless BwdGeom::atomic selects it
  int32_t geom_arg;            // host shapes: the first kernel (count, or the atomic kernel)
                               // reads the geometry from its kernel argument and stores it in
                               // the workspace for the kernels after it
  float lo_g, hi_g;
  uint32_t value_bytes;
  int32_t tile_dots;           // 16-bit values: the tile kernel forms grad_loc / grad_attn from
                               // its staged region rows and a count kernel bins the samples;
                               // else (fp32) the sample-gradient kernel gathers the corner rows
                               // per unit and bins the samples (fp32 rows leave too little LDS
                               // for the region: C2 fp32 backward 430 against 537 us)
  uint32_t grow;               // bytes between the tile kernel's staged grad_out rows (C * s,
                               // value dtype)
  uint32_t vrow;               // bytes between the tile kernel's staged value rows (C * s
                               // rounded up to an odd number of 16-byte slots)
  uint32_t lds_g_bytes;        // bytes of the staged grad_out rows of a sub-batch
  uint32_t lds_bytes;          // total dynamic LDS of the tile kernel
  uint32_t max_chunks;         // upper bound of the chunk count
  uint32_t grid_chunks;        // tile-kernel grid: max_chunks rounded up to a multiple of xcds
  uint32_t xcds;               // XCDs of the device (workgroups are dealt to them round-robin)
  uint64_t grad_loc_elems;     // Bc * Q * H * L * P * dim (NaN fill of invalid shapes)
};

struct BwdBuffers {
  const void* value;
  const void* loc;
  const void* attn;
  const void* grad_out;
  void* grad_value;
  void* grad_loc;
  void* grad_attn;
  uint32_t* counts;      // (groups * bins) x wgpg: per-(tile, bin workgroup) counts -> offsets
  uint32_t* tile_n;      // T: record total of each tile (column scan -> plan)
  uint32_t* bin_start;   // T + 1: first record of each tile
  uint32_t* chunk_off;   // T + 1: first chunk of each tile; [T] = number of chunks
  uint4* chunks;         // max_chunks: {tile, first record, end record, chunks of the tile}
  uint32_t* records;     // record_words(DIM, coordinate bytes) words per record
  float* scratch;        // max_chunks * rcells * C fp32 partials
  float* sums;           // atomic path: fp32 sums in the gathered value's layout
  const BwdGeom* geom;   // level geometry of the launch (written by the first kernel)
};

struct BwdSizes {
  uint64_t counts, tile_n, bin_start, chunk_off, chunk_words, record_words, scratch_floats, sum_floats;
  uint64_t geom_bytes;
  uint64_t total_bytes;
};

// Workspace element counts for a plan, `samples` samples and dimension dim.
BwdSizes bwd_sizes(const BwdPlan& pl, uint64_t samples, int dim, int coord_bytes);

// Clear `bytes` bytes of device memory with a fill kernel (no hipMemset node in graphs).
hipError_t launch_zero_bytes(void* p, size_t bytes, hipStream_t s);

// Enqueue the whole backward for one launch (batch range) on stream s. Its first kernel
// writes bf.geom: a copy of *host_geom, or (host_geom == nullptr) make_geom(*dev_args,
// dev_shapes) computed on the device.
hipError_t run_bwd(const BwdPlan& pl, const BwdGeom* host_geom, const GeomArgs* dev_args,
                   const int32_t* dev_shapes, const BwdBuffers& bf, int dim, int vdt, int cdt,
                   int vec_bytes, hipStream_t s);

bool bwd_supported(int dim, int vdt, int cdt, int vec_bytes);

// Set the thread-local text msda_last_error() returns (printf format) and return `code`.
int set_error(int code, const char* fmt, ...);

// ---------------------------------------------------------------------------------------
// Producer-side kernels of the fused path's backward (msda_fused.hip), for one launch over
// a batch range (units * L * P * 2^dim < 2^31).
struct FusedArgs {
  const float* ref;         // (Bc, Q, L, dim) fp32
  const void* off;          // (Bc, Q, H, L, P, dim) coord dtype
  const void* logits;       // (Bc, Q, H, L, P) coord dtype
  float* loc;               // (Bc, Q, H, L, P, dim) fp32, written by the prep kernel
  float* attn;              // (Bc, Q, H, L, P) fp32, written by the prep kernel
  const float* grad_loc;    // fp32 gradients from the backward kernels
  const float* grad_attn;
  float* grad_ref;          // (Bc, Q, L, dim) fp32
  void* grad_off;           // coord dtype
  void* grad_logits;        // coord dtype
  uint32_t units;           // Bc * Q * H
  uint32_t bq;              // Bc * Q
  int32_t H, L, P;
  int32_t g_log2;           // lanes per unit = 2^g_log2 >= L * P (<= 64), or -1: one thread per unit
  float inv[kMaxLevels][3];   // 1/W, 1/H, 1/D per level (fp32, correctly rounded)
  const int32_t* shapes;    // device (L, dim) shapes, or nullptr: the kernels then compute the
                            // reciprocals from them (as the fused forward does) instead of inv
};

// grad == false: loc and attn from ref, off and logits. grad == true: grad_ref, grad_off and
// grad_logits from grad_loc, grad_attn and attn. cdt is the coord dtype code.
hipError_t launch_fused(const FusedArgs& a, int dim, int cdt, bool grad, hipStream_t s);

}  // namespace msda
