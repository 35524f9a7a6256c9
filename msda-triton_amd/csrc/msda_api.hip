// msda_api.hip — extern "C" entry points declared in include/msda.h.
//
// Host-side work per call: validate the descriptor, pick the kernel instantiation, plan
// the backward's tile geometry (from a host copy of the level shapes, or, for shapes that
// live on the device, from bounds on the host and the shapes on the device), split the batch
// into launches whose byte offsets fit the 32-bit buffer addressing the kernels use, and
// enqueue everything on the caller's stream. No allocation, no synchronisation, no global
// mutable state except the thread-local error text.
#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/msda.h"
#include "msda_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int elem_bytes(int dt) { return dt == MSDA_F32 ? 4 : 2; }

const char* dtype_name(int dt) {
  switch (dt) {
    case MSDA_F32: return "float32";
    case MSDA_F16: return "float16";
    case MSDA_BF16: return "bfloat16";
    default: return "unknown";
  }
}

constexpr uint64_t kLim31 = 0x7FFFFFFFull;
constexpr uint32_t kChunkRecords = 4096;        // records per tile-kernel chunk (rounded to S)
// LDS share of one tile workgroup when n of them share a CU (160 KB LDS per CU)
constexpr uint32_t tile_lds_share(uint32_t n) { return 160u * 1024u / n - 256u; }
constexpr int kMaxBinsLds = 8192;  // bin histogram + bases in 64 KB of LDS

// The current device's compute units, XCDs and per-XCD L2 bytes, which size the staged
// forward's grid, the head-major rule and the XCD-contiguous workgroup mappings. Read once
// per device (hipDeviceGetAttribute); a whole MI355X (256 CUs, 8 XCDs of 4 MB L2) where no
// device answers, e.g. for the host-only workspace queries on a machine without a GPU.
struct Machine {
  uint32_t cus;
  uint32_t xcds;
  uint64_t l2_bytes;  // L2 of one XCD
};

Machine machine() {
  static std::mutex mu;
  static Machine cache[64];
  static bool have[64];
  Machine m{256u, 8u, 4ull << 20};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return m;
  std::lock_guard<std::mutex> lock(mu);
  if (have[dev]) return cache[dev];
  int cus = 0, l2 = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) {
    m.cus = (uint32_t)cus;
    m.xcds = (uint32_t)cus / msda::kCusPerXcd;
    if (m.xcds < 1) m.xcds = 1;
  }
  // the attribute is one XCD's L2 on MI3xx; a figure above 8 MB would be the sum over XCDs
  if (hipDeviceGetAttribute(&l2, hipDeviceAttributeL2CacheSize, dev) == hipSuccess && l2 > 0)
    m.l2_bytes = (uint64_t)l2 > (8ull << 20) ? (uint64_t)l2 / m.xcds : (uint64_t)l2;
  cache[dev] = m;
  have[dev] = true;
  return m;
}

// Lanes per unit and per-lane vector width for one C-channel value row.
struct Layout {
  int vec_bytes;  // bytes per lane per row
  int nvec;       // C / VEC
  int lpu_log2;   // lanes per unit = 2^lpu_log2
  int hg_log2;    // heads whose rows share a 128-byte line
};

bool aligned(const void* p, int a) { return p == nullptr || ((uintptr_t)p % (uintptr_t)a) == 0; }

int choose_layout(const msda_desc* d, const void* const* ptrs, int nptr, Layout* out) {
  const int s = elem_bytes(d->value_dtype);
  const int row = d->channels * s;
  int vb = 16;
  for (; vb >= s; vb /= 2) {
    if (row % vb) continue;
    bool ok = true;
    for (int i = 0; i < nptr; ++i) ok = ok && aligned(ptrs[i], vb);
    if (ok) break;
  }
  if (vb < s)
    return fail(MSDA_ERR_INVALID, "value/output pointers must be aligned to the element size");
  const int nvec = row / vb;
  int lg = 0;
  while ((1 << lg) < nvec) ++lg;
  if (lg > 6)
    return fail(MSDA_ERR_INVALID,
                "channels per head (%d) too large: at most 64 lanes of %d bytes per head row",
                d->channels, vb);
  int hg = 0;
  while (((row << (hg + 1)) <= 128) && (d->num_heads % (1 << (hg + 1)) == 0)) ++hg;
  out->vec_bytes = vb;
  out->nvec = nvec;
  out->lpu_log2 = lg;
  out->hg_log2 = hg;
  return MSDA_OK;
}

int validate(const msda_desc* d) {
  if (!d) return fail(MSDA_ERR_INVALID, "descriptor is NULL");
  if (d->dim != 2 && d->dim != 3) return fail(MSDA_ERR_INVALID, "dim must be 2 or 3, got %d", d->dim);
  if (d->batch < 0 || d->num_keys < 0 || d->num_heads < 1 || d->channels < 1 ||
      d->num_queries < 0 || d->num_levels < 0 || d->num_points < 0)
    return fail(MSDA_ERR_INVALID, "invalid sizes: B=%d K=%lld H=%d C=%d Q=%lld L=%d P=%d",
                d->batch, (long long)d->num_keys, d->num_heads, d->channels,
                (long long)d->num_queries, d->num_levels, d->num_points);
  if (d->value_dtype < MSDA_F32 || d->value_dtype > MSDA_BF16)
    return fail(MSDA_ERR_DTYPE, "value dtype code %d is not fp32, fp16 or bf16", d->value_dtype);
  if (d->coord_dtype != d->value_dtype && d->coord_dtype != MSDA_F32)
    return fail(MSDA_ERR_DTYPE,
                "sampling_locations/attention_weights dtype %s must equal value dtype %s or be "
                "float32",
                dtype_name(d->coord_dtype), dtype_name(d->value_dtype));
  if (d->flags & ~MSDA_FLAG_VALUE_HEAD_MAJOR)
    return fail(MSDA_ERR_INVALID, "unknown flags 0x%x", (unsigned)d->flags);
  if (!isfinite(d->clamp_eps)) return fail(MSDA_ERR_INVALID, "clamp_eps must be finite");
  if (d->num_keys > (int64_t)kLim31)
    return fail(MSDA_ERR_INVALID, "number of keys (%lld) exceeds int32 range",
                (long long)d->num_keys);
  if (d->num_levels > msda::kMaxLevels)
    return fail(MSDA_ERR_INVALID, "at most %d levels are supported, got %d", msda::kMaxLevels,
                d->num_levels);
  const uint64_t lp = (uint64_t)d->num_levels * d->num_points;
  if (lp * d->dim > ((uint64_t)1 << 24))
    return fail(MSDA_ERR_INVALID, "levels*points too large (%llu)", (unsigned long long)lp);
  // One batch must fit one launch: its value bytes (and the fp32 view of them), its lanes,
  // and its backward records stay below 2^31.
  const uint64_t per_b_acc = (uint64_t)d->num_keys * d->num_heads * d->channels * 4ull;
  if (per_b_acc > kLim31)
    return fail(MSDA_ERR_INVALID,
                "value slice of one batch is too large: K*H*C*4 = %llu bytes exceeds 2^31-1",
                (unsigned long long)per_b_acc);
  const uint64_t qh = (uint64_t)d->num_queries * d->num_heads;
  if (qh * 64ull > kLim31)
    return fail(MSDA_ERR_INVALID, "Q*H of one batch too large (%llu units)",
                (unsigned long long)qh);
  if (qh * lp * (1ull << d->dim) > kLim31 || (uint64_t)d->num_queries * d->num_points > kLim31)
    return fail(MSDA_ERR_INVALID, "Q*H*L*P of one batch too large for the backward");
  return MSDA_OK;
}

int64_t min64(int64_t a, int64_t b) { return a < b ? a : b; }

// Batches per launch such that every 32-bit in-kernel offset stays below 2^31.
int64_t batches_per_launch(const msda_desc* d, const Layout& lay) {
  const uint64_t per_b_acc = (uint64_t)d->num_keys * d->num_heads * d->channels * 4ull;
  const uint64_t qh = (uint64_t)d->num_queries * d->num_heads;
  const uint64_t per_b_lanes = qh << lay.lpu_log2;
  const uint64_t per_b_rec = qh * d->num_levels * d->num_points * (1ull << d->dim);
  int64_t nb = d->batch;
  if (per_b_acc) nb = min64(nb, (int64_t)(kLim31 / per_b_acc));
  if (per_b_lanes) nb = min64(nb, (int64_t)(kLim31 / per_b_lanes));
  if (per_b_rec) nb = min64(nb, (int64_t)(kLim31 / per_b_rec));
  return nb < 1 ? 1 : nb;
}

// Whether the kernels should gather from a head-major (B, H, K, C) copy of value. In the
// (B, K, H, C) layout a row shorter than a 128-byte line shares its line with other heads,
// and a head's rows touch K lines; once those exceed an XCD's L2, random gathers miss on
// most lines. In the copy one head's rows are contiguous (half the footprint for 64-byte
// rows) and the two x-neighbours of a corner pair often share a line. The copy costs a read
// and a write of value, so it is made only when the gathers are many times larger.
bool use_head_major(const msda_desc* d) {
  const uint64_t row = (uint64_t)d->channels * elem_bytes(d->value_dtype);
  const uint64_t gathers = (uint64_t)d->num_queries * d->num_levels * d->num_points << d->dim;
  return d->num_heads > 1 && row <= 64 && (uint64_t)d->num_keys * 128 > machine().l2_bytes &&
         gathers >= 8 * (uint64_t)d->num_keys;
}

void fill_params(const msda_desc* d, const Layout& lay, int64_t nb, msda::Params* p) {
  const uint32_t Q = (uint32_t)d->num_queries, H = (uint32_t)d->num_heads;
  p->K = (int32_t)d->num_keys;
  p->H = d->num_heads;
  p->C = d->channels;
  p->L = d->num_levels;
  p->P = d->num_points;
  p->Q = Q;
  p->num_units = (uint32_t)(nb * Q * H);
  p->div_qh = msda::make_fastdiv(Q * H);
  p->div_qhg = msda::make_fastdiv(Q << lay.hg_log2);
  p->hg_log2 = lay.hg_log2;
  p->lpu_log2 = lay.lpu_log2;
  p->nvec = lay.nvec;
  p->clamp = d->clamp_grid ? 1 : 0;
  // torch.clamp(min=-1+eps, max=1-eps) converts the Python-double bounds to the tensor dtype.
  p->lo_g = (float)(-1.0 + d->clamp_eps);
  p->hi_g = (float)(1.0 - d->clamp_eps);
  const uint64_t lanes = (uint64_t)p->num_units << lay.lpu_log2;
  p->nblocks = (uint32_t)((lanes + msda::kBlock - 1) / msda::kBlock);
  p->xcds = machine().xcds;
  p->value_bytes = (uint32_t)(nb * (uint64_t)d->num_keys * H * d->channels * elem_bytes(d->value_dtype));
}

// ---------------------------------------------------------------------------------------
// Backward plan. With host shapes every size is exact; without them (device-resident
// shapes) the bin capacity is estimated from K and the launch falls back, on the device,
// to the atomic grad_value path when the levels need more bins.
struct BwdHostPlan {
  msda::BwdPlan pl;
  msda::BwdSizes sz;
  msda::GeomArgs ga;  // make_geom inputs (groups of a full launch)
  Layout lay;
  int64_t nb;
};

// Upper estimate of a pyramid's tiles from K alone: 1.5x the tiles its cells fill, plus a
// few partial tiles per level. Levels that are thin along one axis can need more; their
// launches take the atomic path on the device.
int64_t estimate_tiles(const msda_desc* d, int cells) {
  const int64_t area = ((int64_t)d->num_keys + cells - 1) / cells;
  return area + area / 2 + 4 * ((int64_t)1 << d->dim) * d->num_levels + 64;
}

int plan_bwd(const msda_desc* d, const int32_t* hs, const void* const* ptrs, int nptr,
             BwdHostPlan* out) {
  memset(out, 0, sizeof(*out));
  msda::BwdPlan& pl = out->pl;
  const bool dev = hs == nullptr;  // planned without the shapes
  int64_t total = 0;
  for (int l = 0; l < d->num_levels && !dev; ++l) {
    int64_t n = 1;
    for (int k = 0; k < d->dim; ++k) {
      const int32_t v = hs[l * d->dim + k];
      if (v < 0) return fail(MSDA_ERR_INVALID, "spatial shape of level %d is negative", l);
      n *= v;
    }
    total += n;
    if (total > (int64_t)kLim31) return fail(MSDA_ERR_INVALID, "Total number of keys exceeds int32 range");
  }
  if (!dev && total != d->num_keys)
    return fail(MSDA_ERR_INVALID,
                "value dim 1 (%lld) does not match sum of spatial shapes (%lld)",
                (long long)d->num_keys, (long long)total);
  // The backward's per-lane width depends on C only (never on pointer alignment), so the
  // plan and the workspace size are the same with or without pointers.
  const void* none[1] = {nullptr};
  int rc = choose_layout(d, none, 0, &out->lay);
  if (rc) return rc;
  const Layout& lay = out->lay;
  for (int i = 0; i < nptr; ++i)
    if (!aligned(ptrs[i], lay.vec_bytes))
      return fail(MSDA_ERR_INVALID, "msda_bwd: tensor pointers must be %d-byte aligned",
                  lay.vec_bytes);
  const int s = elem_bytes(d->value_dtype);
  const int nc = 1 << d->dim;
  // records name their sample by q * P + p in 27 bits
  const bool ids_fit = (uint64_t)d->num_queries * d->num_points <= (uint64_t)msda::kRecIdMask;
  // Tile extents and sub-batch size: start from 16x16 (2D) / 8x8x8 (3D) cells and
  // S = kTileThreads<dim> records (one per thread); halve the largest tile extent until a thread
  // owns at most tile_max_items (region cell, owner chunk) items, and lower S in steps of
  // half a wave until the sub-batch's grad_out rows, sorted entries, two counter sets and the
  // region's value rows fit the LDS share of one workgroup. Fewer records per sub-batch cost
  // more than fewer workgroups per CU (C2 tile kernel: S = 160 at four workgroups per CU
  // 213 us, S = 224 161 us), so S stays at half the threads or more: the LDS share is that
  // of four, three or two workgroups per CU (2D; two in 3D), then of one, and only then do
  // the tiles shrink for LDS.
  const uint32_t NT = d->dim == 2 ? msda::kTileThreads<2> : msda::kTileThreads<3>;
  // 16-bit values: the tile kernel forms the sample gradients from staged region rows
  const bool tile_dots = s == 2;
  // staged rows, both in the value dtype: grad_out rows C * s bytes apart; value rows C * s
  // rounded up to an odd number of 16-byte slots, so one chunk of random rows spreads over
  // every bank slot (C2 tile kernel 237 -> 224 us). Padding the grad_out rows too spreads
  // the dot products' reads of consecutive records' rows, but the LDS it takes lowers S
  // (2D 256 -> 224, 3D 448 -> 416) and that costs more (224 -> 229 us, C5 653 -> 669 us).
  const uint32_t grow = (uint32_t)(d->channels * s);
  const uint32_t vrow = tile_dots ? ((uint32_t)(d->channels * s) + 15u) / 32u * 32u + 16u : 0u;
  const int ov = msda::tile_owner_vec(lay.vec_bytes / s, s);
  const int onv = d->channels / ov;
  int T[3];
  uint32_t S = NT, lds = 0;
  int rcells = 0;
  auto shrink = [&]() {
    const int k = (T[2] >= T[1] && T[2] >= T[0] && T[2] > 1) ? 2 : (T[1] >= T[0] && T[1] > 1 ? 1 : 0);
    if (T[k] <= 1) return false;
    T[k] /= 2;
    return true;
  };
  // largest tile, then largest S >= smin, that meets the per-thread limit and the LDS
  // budget; shrink: smaller tiles when no S fits
  auto fit = [&](uint32_t budget, uint32_t smin, bool shrink_for_lds) {
    T[0] = T[1] = 16;
    T[2] = 1;
    if (d->dim == 3) T[0] = T[1] = T[2] = 8;
    S = NT;
    for (;;) {
      const int rz = d->dim == 3 ? T[2] + 1 : 1;
      rcells = (T[0] + 1) * (T[1] + 1) * rz;
      const int mi = msda::tile_max_items(ov);
      if ((uint64_t)rcells * onv > (uint64_t)mi * NT) {
        if (!shrink()) return false;
        continue;
      }
      lds = S * grow + S * nc * 8u + 2u * (uint32_t)((rcells + 4) & ~3) * 4u +
            (uint32_t)rcells * vrow;
      // a corner's (cell, rank) pair is packed into 16 + 16 bits
      if (rcells >= (1 << 16) || S * nc >= (1u << 16)) {
        if (!shrink()) return false;
        continue;
      }
      if (lds <= budget) return true;
      // (steps of 32 records: C2 S = 224 against 192 in steps of 64, backward 358 -> 348 us)
      if (S >= smin + 32u) {
        S -= 32u;
        continue;
      }
      if (!shrink_for_lds || !shrink()) return false;
      S = NT;
    }
  };
  bool planned = false;
  if (d->dim == 2) {
    for (uint32_t wgs = 4; wgs >= 2 && !planned; --wgs)
      planned = fit(tile_lds_share(wgs), NT / 2, false);
  } else {
    planned = fit(tile_lds_share(2), NT / 2, false);
  }
  if (!planned) planned = fit(tile_lds_share(1), 32u, true);
  if (!planned)
    return fail(MSDA_ERR_INVALID, "channels per head (%d) too large for the backward", d->channels);
  pl.TX = T[0];
  pl.TY = T[1];
  pl.TZ = T[2];
  auto log2i = [](int v) {
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
  };
  pl.tx_log2 = log2i(T[0]);
  pl.ty_log2 = log2i(T[1]);
  pl.tz_log2 = log2i(T[2]);
  pl.div_nvec = msda::make_fastdiv((uint32_t)lay.nvec);
  pl.onv = onv;
  pl.div_onv = msda::make_fastdiv((uint32_t)onv);
  pl.div_tx = msda::make_fastdiv((uint32_t)T[0]);
  pl.div_txy = msda::make_fastdiv((uint32_t)(T[0] * T[1]));
  pl.RX = T[0] + 1;
  pl.RY = T[1] + 1;
  pl.RZ = d->dim == 3 ? T[2] + 1 : 1;
  pl.cells = T[0] * T[1] * T[2];
  pl.rcells = rcells;
  pl.S = S;
  pl.tile_dots = tile_dots ? 1 : 0;
  pl.grow = grow;
  pl.vrow = vrow;
  pl.lds_g_bytes = S * grow;
  pl.lds_bytes = lds;
  // Tiles per head over all levels: exact from host shapes, else an estimate from K.
  // Levels with more than kMaxBinsLds tiles per head do not fit the LDS binning of the
  // count and fill kernels, and more than 2^27 samples per (b, h, level) do not fit a record
  // id: such plans scatter grad_value with fp32 atomics instead (atomic kernel, then one
  // rounding pass).
  int64_t tiles = 0;
  for (int l = 0; l < d->num_levels && !dev; ++l) {
    const int32_t* r = hs + l * d->dim;
    const int32_t W = r[d->dim - 1], H = r[d->dim - 2], D = d->dim == 3 ? r[0] : 1;
    tiles += (int64_t)msda::tiles_along(W, pl.TX) * msda::tiles_along(H, pl.TY) *
             msda::tiles_along(D, pl.TZ);
  }
  if (dev) tiles = estimate_tiles(d, pl.cells);
  const bool atomic = (!dev && tiles > kMaxBinsLds) || !ids_fit;
  pl.static_atomic = atomic ? 1 : 0;
  pl.fallback = dev && !atomic ? 1 : 0;
  if (atomic) tiles = 0;
  // value already head-major (MSDA_FLAG_VALUE_HEAD_MAJOR): read it in that layout
  const bool head_major = (d->flags & MSDA_FLAG_VALUE_HEAD_MAJOR) != 0;
  // Heads whose rows share 128-byte lines are grouped (their units and chunks run on one
  // XCD). Where a head's keys exceed an XCD's L2 (the forward's head-major rule), one head
  // per group keeps one head's grad_out rows per XCD instead (C5: tile 699 -> 523 us).
  int hg = head_major || (!atomic && use_head_major(d)) ? 0 : lay.hg_log2;
  while (hg > 0 && (tiles << hg) > kMaxBinsLds) --hg;
  const int64_t bins_cap = (tiles << hg) < kMaxBinsLds ? (tiles << hg) : kMaxBinsLds;
  pl.L = d->num_levels;
  pl.P = d->num_points;
  pl.C = d->channels;
  pl.H = d->num_heads;
  pl.K = (int32_t)d->num_keys;
  pl.Q = (uint32_t)d->num_queries;
  pl.div_p = msda::make_fastdiv((uint32_t)(d->num_points > 0 ? d->num_points : 1));
  pl.div_lp = msda::make_fastdiv((uint32_t)(d->num_levels * d->num_points > 0
                                                ? d->num_levels * d->num_points : 1));
  pl.head_major = head_major ? 1 : 0;
  pl.hg_log2 = hg;
  pl.bins_cap = (int32_t)bins_cap;
  pl.upw = (msda::kGradThreads >> lay.lpu_log2) * msda::kGradRounds;
  if (d->dim == 3) {
    const uint64_t upw2 = 2u * (uint64_t)pl.upw;
    const uint64_t wgs2 = (uint64_t)(((uint64_t)d->batch * d->num_heads) >> hg) *
                          ((((uint64_t)d->num_queries << hg) + upw2 - 1) / upw2);
    if (wgs2 >= (uint64_t)msda::kGradWgsPerCu * machine().cus) pl.upw = (int32_t)upw2;
  }
  pl.wgpg = (int32_t)((((uint64_t)d->num_queries << hg) + pl.upw - 1) / pl.upw);
  pl.R = (kChunkRecords + pl.S - 1) / pl.S * pl.S;
  pl.lpu_log2 = lay.lpu_log2;
  pl.nvec = lay.nvec;
  pl.clamp = d->clamp_grid ? 1 : 0;
  pl.lo_g = (float)(-1.0 + d->clamp_eps);
  pl.hi_g = (float)(1.0 - d->clamp_eps);
  int64_t nb = batches_per_launch(d, lay);
  // the per-(bin workgroup, tile) count matrix must stay below 2^31 entries too
  const uint64_t per_b_counts = (uint64_t)(d->num_heads >> hg) * bins_cap * (uint64_t)pl.wgpg;
  if (per_b_counts > kLim31) return fail(MSDA_ERR_INVALID, "backward count matrix too large");
  if (per_b_counts) nb = min64(nb, (int64_t)(kLim31 / per_b_counts));
  if (nb < 1) nb = 1;
  out->nb = nb;
  pl.groups = (int32_t)((nb * d->num_heads) >> hg);
  pl.T_cap = (uint32_t)pl.groups * (uint32_t)bins_cap;
  const uint64_t samples =
      (uint64_t)nb * d->num_queries * d->num_heads * d->num_levels * d->num_points;
  pl.max_chunks = atomic ? 0u : pl.T_cap + (uint32_t)((samples + pl.R - 1) / pl.R);
  pl.xcds = machine().xcds;
  pl.grid_chunks = (pl.max_chunks + pl.xcds - 1) / pl.xcds * pl.xcds;
  pl.value_bytes = (uint32_t)(nb * (uint64_t)d->num_keys * d->num_heads * d->channels * s);
  pl.grad_loc_elems = samples * (uint64_t)d->dim;
  out->sz = msda::bwd_sizes(pl, samples, d->dim, elem_bytes(d->coord_dtype));
  msda::GeomArgs& ga = out->ga;
  ga.dim = d->dim;
  ga.L = d->num_levels;
  ga.H = d->num_heads;
  ga.C = d->channels;
  ga.s = s;
  ga.head_major = pl.head_major;
  ga.hg_log2 = hg;
  ga.groups = pl.groups;
  ga.TX = pl.TX;
  ga.TY = pl.TY;
  ga.TZ = pl.TZ;
  ga.bins_cap = (int32_t)bins_cap;
  ga.static_atomic = pl.static_atomic;
  ga.K = d->num_keys;
  if (!msda::bwd_supported(d->dim, d->value_dtype, d->coord_dtype, lay.vec_bytes))
    return fail(MSDA_ERR_DTYPE, "no backward kernel for this dtype combination");
  return MSDA_OK;
}

void carve(char* ws, const msda::BwdSizes& z, msda::BwdBuffers* bf) {
  auto al = [](uint64_t b) { return (b + 255) & ~(uint64_t)255; };
  char* p = ws;
  bf->geom = reinterpret_cast<const msda::BwdGeom*>(p);
  p += al(z.geom_bytes);
  bf->counts = reinterpret_cast<uint32_t*>(p);
  p += al(z.counts * 4);
  bf->tile_n = reinterpret_cast<uint32_t*>(p);
  p += al(z.tile_n * 4);
  bf->bin_start = reinterpret_cast<uint32_t*>(p);
  p += al(z.bin_start * 4);
  bf->chunk_off = reinterpret_cast<uint32_t*>(p);
  p += al(z.chunk_off * 4);
  bf->chunks = reinterpret_cast<uint4*>(p);
  p += al(z.chunk_words * 4);
  bf->records = reinterpret_cast<uint32_t*>(p);
  p += al(z.record_words * 4);
  bf->scratch = reinterpret_cast<float*>(p);
  p += al(z.scratch_floats * 4);
  bf->sums = reinterpret_cast<float*>(p);
}

// Body of msda_fwd and msda_fwd_fused. fused: `loc` / `attn` are the sampling offsets and
// attention logits and `ref` the fp32 reference points; the kernels form the locations and
// weights themselves.
int fwd_impl(const msda_desc* d, const void* value, const int32_t* spatial_shapes,
             const int32_t* level_start, const void* sampling_locations,
             const void* attention_weights, const float* ref, void* output, void* workspace,
             size_t workspace_bytes, void* stream, bool fused) {
  if (d && d->flags) return fail(MSDA_ERR_INVALID, "forward: flags apply to the backward only");
  const char* name = fused ? "msda_fwd_fused" : "msda_fwd";
  int rc = validate(d);
  if (rc) return rc;
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  if (units == 0) return MSDA_OK;
  const bool has_samples = d->num_levels > 0 && d->num_points > 0;
  if (!output || (d->num_keys > 0 && !value) ||
      (has_samples && (!sampling_locations || !attention_weights || (fused && !ref))) ||
      (d->num_levels > 0 && (!spatial_shapes || !level_start)))
    return fail(MSDA_ERR_INVALID, "%s: required pointer is NULL", name);
  const void* vptrs[2] = {value, output};
  Layout lay;
  if ((rc = choose_layout(d, vptrs, 2, &lay))) return rc;
  msda::LaunchFn fn = msda::get_fwd_launcher(d->dim, d->value_dtype, d->coord_dtype, lay.vec_bytes, false, fused);
  msda::LaunchFn fn_staged =
      msda::get_fwd_launcher(d->dim, d->value_dtype, d->coord_dtype, lay.vec_bytes, true, fused);
  if (!fn || !fn_staged) return fail(MSDA_ERR_DTYPE, "no forward kernel for this dtype combination");

  const int64_t nb = batches_per_launch(d, lay);
  const int sv = elem_bytes(d->value_dtype), sc = elem_bytes(d->coord_dtype);
  const uint64_t LP = (uint64_t)d->num_levels * d->num_points;
  const uint64_t qh = (uint64_t)d->num_queries * d->num_heads;
  const uint64_t kv = (uint64_t)d->num_keys * d->num_heads * d->channels;
  for (int64_t b0 = 0; b0 < d->batch; b0 += nb) {
    const int64_t bc = (d->batch - b0) < nb ? (d->batch - b0) : nb;
    msda::Params p{};
    fill_params(d, lay, bc, &p);
    p.value = static_cast<const char*>(value) + (uint64_t)b0 * kv * sv;
    p.loc = static_cast<const char*>(sampling_locations) + (uint64_t)b0 * qh * LP * d->dim * sc;
    p.attn = static_cast<const char*>(attention_weights) + (uint64_t)b0 * qh * LP * sc;
    p.out = static_cast<char*>(output) + (uint64_t)b0 * qh * d->channels * sv;
    p.shapes = spatial_shapes;
    p.starts = level_start;
    p.ref = fused ? ref + (uint64_t)b0 * d->num_queries * d->num_levels * d->dim : nullptr;
    p.coords_aligned = aligned(p.loc, 16) && aligned(p.attn, 16);
    // head-major copy of this launch's value slice when it pays and the workspace holds it
    const uint64_t vbytes = (uint64_t)bc * kv * sv;
    if (use_head_major(d) && workspace && workspace_bytes >= vbytes &&
        aligned(workspace, lay.vec_bytes)) {
      hipError_t e = msda::launch_head_major(p.value, workspace, (uint32_t)bc, (uint32_t)d->num_keys,
                                             (uint32_t)d->num_heads, (uint32_t)(d->channels * sv),
                                             lay.vec_bytes, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) return fail(MSDA_ERR_HIP, "%s relayout failed: %s", name, hipGetErrorString(e));
      p.value_h = workspace;
    }
    // Staged kernel: one workgroup per CU, each (batch, head) slice split into query
    // ranges; used when every workgroup gets enough queries to amortise its LDS copy.
    const uint64_t slices = (uint64_t)bc * d->num_heads;
    const uint64_t cus = machine().cus;
    const uint64_t splits = (cus + slices - 1) / slices;
    const uint64_t qper = ((uint64_t)d->num_queries + splits - 1) / splits;
    // the LDS holds at least one staged row beside the all-zero row
    const bool staged = has_samples && qper >= msda::kFwdStageMinQueries &&
                        (uint64_t)d->channels * sv * 2 <= msda::kFwdStageLds;
    if (staged) {
      p.splits = (uint32_t)splits;
      p.qper = (uint32_t)qper;
      p.stage_bytes = msda::kFwdStageLds;
      p.nblocks = (uint32_t)(slices * splits);
    }
    hipError_t e = (staged ? fn_staged : fn)(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(MSDA_ERR_HIP, "%s launch failed: %s", name, hipGetErrorString(e));
  }
  return MSDA_OK;
}


// Workspace of msda_bwd_fused: fp32 loc, attn, grad_loc, grad_attn, then the workspace of
// the inner msda_bwd over those fp32 tensors (coord dtype float32). Byte offsets.
struct FusedWs {
  uint64_t loc, attn, gloc, gattn;
  uint64_t inner, inner_bytes;  // the inner msda_bwd workspace
  uint64_t total;
};

// hs == nullptr: the inner backward is planned without the shapes (msda_bwd_dev).
bool fused_ws(const msda_desc* d, const int32_t* hs, FusedWs* w) {
  auto al = [](uint64_t b) { return (b + 255) & ~(uint64_t)255; };
  msda_desc d32 = *d;
  d32.coord_dtype = MSDA_F32;
  const uint64_t samples = (uint64_t)d->batch * d->num_queries * d->num_heads * d->num_levels * d->num_points;
  BwdHostPlan hp;
  const void* none[1] = {nullptr};
  if (plan_bwd(&d32, hs, none, 0, &hp)) return false;
  w->loc = 0;
  w->attn = w->loc + al(samples * d->dim * 4);
  w->gloc = w->attn + al(samples * 4);
  w->gattn = w->gloc + al(samples * d->dim * 4);
  w->inner = w->gattn + al(samples * 4);
  w->inner_bytes = hp.sz.total_bytes;
  w->total = w->inner + al(w->inner_bytes);
  return true;
}

// Fused-path prep / grad launches over batch ranges that keep every index 32-bit. The
// reciprocals of the level extents come from the host shapes hs, or (hs == nullptr) are
// computed by the kernels from the device shapes ds.
int run_fused_kernels(const msda_desc* d, const int32_t* hs, const int32_t* ds,
                      msda::FusedArgs a, bool grad, hipStream_t st) {
  Layout lay;
  const void* none[1] = {nullptr};
  int rc = choose_layout(d, none, 0, &lay);
  if (rc) return rc;
  a.shapes = hs ? nullptr : ds;
  for (int l = 0; l < d->num_levels && hs; ++l) {
    const int32_t* r = hs + l * d->dim;
    // the forward kernel's reciprocals: 1.0f / (float)extent, correctly rounded on both sides
    a.inv[l][0] = 1.0f / (float)r[d->dim - 1];                   // W
    a.inv[l][1] = 1.0f / (float)r[d->dim - 2];                   // H
    a.inv[l][2] = 1.0f / (d->dim == 3 ? (float)r[0] : 1.0f);     // D
  }
  a.H = d->num_heads;
  a.L = d->num_levels;
  a.P = d->num_points;
  const int64_t lp = (int64_t)d->num_levels * d->num_points;
  a.g_log2 = -1;
  if (lp <= 64) {
    a.g_log2 = 0;
    while ((1 << a.g_log2) < lp) ++a.g_log2;
  }
  const int64_t nb = batches_per_launch(d, lay);
  const int sc = elem_bytes(d->coord_dtype);
  const uint64_t LP = (uint64_t)d->num_levels * d->num_points;
  const uint64_t qh = (uint64_t)d->num_queries * d->num_heads;
  const uint64_t nref = (uint64_t)d->num_queries * d->num_levels * d->dim;  // per batch
  const uint64_t nloc = qh * LP * d->dim, natt = qh * LP;                    // per batch
  for (int64_t b0 = 0; b0 < d->batch; b0 += nb) {
    const int64_t bc = (d->batch - b0) < nb ? (d->batch - b0) : nb;
    msda::FusedArgs x = a;
    x.units = (uint32_t)(bc * qh);
    x.bq = (uint32_t)(bc * d->num_queries);
    x.ref = a.ref ? a.ref + b0 * nref : nullptr;
    x.off = a.off ? static_cast<const char*>(a.off) + b0 * nloc * sc : nullptr;
    x.logits = a.logits ? static_cast<const char*>(a.logits) + b0 * natt * sc : nullptr;
    x.loc = a.loc + b0 * nloc;
    x.attn = a.attn + b0 * natt;
    x.grad_loc = a.grad_loc ? a.grad_loc + b0 * nloc : nullptr;
    x.grad_attn = a.grad_attn ? a.grad_attn + b0 * natt : nullptr;
    x.grad_ref = a.grad_ref ? a.grad_ref + b0 * nref : nullptr;
    x.grad_off = a.grad_off ? static_cast<char*>(a.grad_off) + b0 * nloc * sc : nullptr;
    x.grad_logits = a.grad_logits ? static_cast<char*>(a.grad_logits) + b0 * natt * sc : nullptr;
    hipError_t e = msda::launch_fused(x, d->dim, d->coord_dtype, grad, st);
    if (e != hipSuccess)
      return fail(MSDA_ERR_HIP, "msda_bwd_fused %s launch failed: %s", grad ? "grad" : "prep",
                  hipGetErrorString(e));
  }
  return MSDA_OK;
}
// Body of msda_bwd (hs: host shapes) and msda_bwd_dev (hs == nullptr, ds: device shapes).
int bwd_impl(const msda_desc* d, const int32_t* hs, const int32_t* ds, const void* value,
             const void* sampling_locations, const void* attention_weights,
             const void* grad_output, void* grad_value, void* grad_sampling_locations,
             void* grad_attention_weights, void* workspace, size_t workspace_bytes,
             void* stream, const char* name) {
  int rc = validate(d);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int sv = elem_bytes(d->value_dtype);
  const size_t nval = (size_t)d->batch * (size_t)d->num_keys * d->num_heads * d->channels;
  if (nval && !grad_value) return fail(MSDA_ERR_INVALID, "%s: grad_value is NULL", name);
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  if (units == 0 || d->num_levels == 0 || d->num_points == 0) {
    // no samples: grad_value is zero, the other gradients are empty
    hipError_t e = msda::launch_zero_bytes(grad_value, nval * sv, st);
    if (e != hipSuccess) return fail(MSDA_ERR_HIP, "%s clear failed: %s", name, hipGetErrorString(e));
    return MSDA_OK;
  }
  if ((d->num_keys > 0 && !value) || !sampling_locations || !attention_weights || !grad_output ||
      !grad_sampling_locations || !grad_attention_weights || (!hs && !ds))
    return fail(MSDA_ERR_INVALID, "%s: required pointer is NULL", name);
  const void* vptrs[3] = {value, grad_output, grad_value};
  BwdHostPlan hp;
  if ((rc = plan_bwd(d, hs, vptrs, 3, &hp))) return rc;
  if (!workspace || workspace_bytes < hp.sz.total_bytes)
    return fail(MSDA_ERR_WORKSPACE, "%s needs %llu workspace bytes, got %zu", name,
                (unsigned long long)hp.sz.total_bytes, workspace_bytes);
  if (((uintptr_t)workspace % 256) != 0)
    return fail(MSDA_ERR_INVALID, "%s: workspace must be 256-byte aligned", name);

  const int sc = elem_bytes(d->coord_dtype);
  const uint64_t LP = (uint64_t)d->num_levels * d->num_points;
  const uint64_t qh = (uint64_t)d->num_queries * d->num_heads;
  const uint64_t kv = (uint64_t)d->num_keys * d->num_heads * d->channels;
  msda::BwdBuffers bf{};
  carve(static_cast<char*>(workspace), hp.sz, &bf);
  msda::BwdGeom geom;
  for (int64_t b0 = 0; b0 < d->batch; b0 += hp.nb) {
    const int64_t bc = (d->batch - b0) < hp.nb ? (d->batch - b0) : hp.nb;
    msda::BwdPlan pl = hp.pl;
    msda::GeomArgs ga = hp.ga;
    pl.groups = (int32_t)((bc * d->num_heads) >> pl.hg_log2);
    pl.T_cap = (uint32_t)pl.groups * (uint32_t)pl.bins_cap;
    pl.value_bytes = (uint32_t)(bc * kv * sv);
    pl.grad_loc_elems = (uint64_t)bc * qh * LP * d->dim;
    ga.groups = pl.groups;
    if (hs) make_geom(ga, hs, &geom);
    bf.value = static_cast<const char*>(value) + (uint64_t)b0 * kv * sv;
    bf.loc = static_cast<const char*>(sampling_locations) + (uint64_t)b0 * qh * LP * d->dim * sc;
    bf.attn = static_cast<const char*>(attention_weights) + (uint64_t)b0 * qh * LP * sc;
    bf.grad_out = static_cast<const char*>(grad_output) + (uint64_t)b0 * qh * d->channels * sv;
    bf.grad_value = static_cast<char*>(grad_value) + (uint64_t)b0 * kv * sv;
    bf.grad_loc = static_cast<char*>(grad_sampling_locations) + (uint64_t)b0 * qh * LP * d->dim * sc;
    bf.grad_attn = static_cast<char*>(grad_attention_weights) + (uint64_t)b0 * qh * LP * sc;
    pl.coords_aligned = aligned(bf.loc, 16) && aligned(bf.attn, 16) && aligned(bf.grad_loc, 16) &&
                        aligned(bf.grad_attn, 16);
    hipError_t e = msda::run_bwd(pl, hs ? &geom : nullptr, hs ? nullptr : &ga, ds, bf, d->dim,
                                 d->value_dtype, d->coord_dtype, hp.lay.vec_bytes, st);
    if (e != hipSuccess) return fail(MSDA_ERR_HIP, "%s launch failed: %s", name, hipGetErrorString(e));
  }
  return MSDA_OK;
}

// Body of msda_bwd_fused (hs: host shapes) and msda_bwd_fused_dev (hs == nullptr, ds:
// device shapes).
int fused_bwd_impl(const msda_desc* d, const int32_t* hs, const int32_t* ds, const void* value,
                   const float* reference_points, const void* sampling_offsets,
                   const void* attention_logits, const void* grad_output, void* grad_value,
                   float* grad_reference_points, void* grad_sampling_offsets,
                   void* grad_attention_logits, void* workspace, size_t workspace_bytes,
                   void* stream, const char* name) {
  int rc = validate(d);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  const uint64_t nref = (uint64_t)d->batch * d->num_queries * d->num_levels * d->dim;
  if (units == 0 || d->num_levels == 0 || d->num_points == 0) {
    // no samples: grad_value and grad_reference_points are zero, the others empty
    const size_t nval = (size_t)d->batch * (size_t)d->num_keys * d->num_heads * d->channels;
    if ((nval && !grad_value) || (nref && !grad_reference_points))
      return fail(MSDA_ERR_INVALID, "%s: required pointer is NULL", name);
    hipError_t e = msda::launch_zero_bytes(grad_value, nval * elem_bytes(d->value_dtype), st);
    if (e == hipSuccess) e = msda::launch_zero_bytes(grad_reference_points, nref * 4, st);
    if (e != hipSuccess) return fail(MSDA_ERR_HIP, "%s clear failed: %s", name, hipGetErrorString(e));
    return MSDA_OK;
  }
  if (!reference_points || !sampling_offsets || !attention_logits || !grad_reference_points ||
      !grad_sampling_offsets || !grad_attention_logits || (!hs && !ds))
    return fail(MSDA_ERR_INVALID, "%s: required pointer is NULL", name);
  FusedWs w;
  if (!fused_ws(d, hs, &w)) return MSDA_ERR_INVALID;
  if (!workspace || workspace_bytes < w.total)
    return fail(MSDA_ERR_WORKSPACE, "%s needs %llu workspace bytes, got %zu", name,
                (unsigned long long)w.total, workspace_bytes);
  if (((uintptr_t)workspace % 256) != 0)
    return fail(MSDA_ERR_INVALID, "%s: workspace must be 256-byte aligned", name);
  char* ws = static_cast<char*>(workspace);
  msda::FusedArgs a{};
  a.ref = reference_points;
  a.off = sampling_offsets;
  a.logits = attention_logits;
  a.loc = reinterpret_cast<float*>(ws + w.loc);
  a.attn = reinterpret_cast<float*>(ws + w.attn);
  // 1. the forward's fp32 locations and weights
  if ((rc = run_fused_kernels(d, hs, ds, a, false, st))) return rc;
  // 2. the ordinary backward on them
  msda_desc d32 = *d;
  d32.coord_dtype = MSDA_F32;
  float* gloc = reinterpret_cast<float*>(ws + w.gloc);
  float* gattn = reinterpret_cast<float*>(ws + w.gattn);
  rc = bwd_impl(&d32, hs, ds, value, a.loc, a.attn, grad_output, grad_value, gloc, gattn,
                ws + w.inner, w.inner_bytes, stream, name);
  if (rc) return rc;
  // 3. through the location and softmax formation
  a.grad_loc = gloc;
  a.grad_attn = gattn;
  a.grad_ref = grad_reference_points;
  a.grad_off = grad_sampling_offsets;
  a.grad_logits = grad_attention_logits;
  return run_fused_kernels(d, hs, ds, a, true, st);
}

}  // namespace

namespace msda {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace msda

extern "C" {

int msda_abi_version(void) { return MSDA_ABI_VERSION; }

const char* msda_last_error(void) { return g_err; }

int msda_validate(const msda_desc* desc) {
  g_err[0] = 0;
  return validate(desc);
}

size_t msda_fwd_workspace_bytes(const msda_desc* d) {
  g_err[0] = 0;
  if (validate(d)) return 0;
  if (d->flags) return fail(MSDA_ERR_INVALID, "msda_fwd_workspace_bytes: flags apply to the backward only"), 0;
  if (!use_head_major(d) || d->batch == 0 || d->num_queries == 0) return 0;
  Layout lay;
  const void* none[1] = {nullptr};
  if (choose_layout(d, none, 0, &lay)) return 0;
  const int64_t nb = batches_per_launch(d, lay);
  const int64_t bmax = d->batch < nb ? d->batch : nb;
  return (size_t)bmax * (size_t)d->num_keys * d->num_heads * d->channels * elem_bytes(d->value_dtype);
}

int msda_fwd(const msda_desc* d, const void* value, const int32_t* spatial_shapes,
             const int32_t* level_start, const void* sampling_locations,
             const void* attention_weights, void* output, void* workspace,
             size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return fwd_impl(d, value, spatial_shapes, level_start, sampling_locations, attention_weights,
                  nullptr, output, workspace, workspace_bytes, stream, false);
}

int msda_fwd_fused(const msda_desc* d, const void* value, const int32_t* spatial_shapes,
                   const int32_t* level_start, const float* reference_points,
                   const void* sampling_offsets, const void* attention_logits, void* output,
                   void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return fwd_impl(d, value, spatial_shapes, level_start, sampling_offsets, attention_logits,
                  reference_points, output, workspace, workspace_bytes, stream, true);
}

size_t msda_bwd_workspace_bytes(const msda_desc* d, const int32_t* host_spatial_shapes) {
  g_err[0] = 0;
  if (validate(d)) return 0;
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  if (units == 0 || d->num_levels == 0 || d->num_points == 0) return 0;
  if (!host_spatial_shapes) return fail(MSDA_ERR_INVALID, "host spatial shapes are NULL"), 0;
  BwdHostPlan hp;
  const void* none[1] = {nullptr};
  if (plan_bwd(d, host_spatial_shapes, none, 0, &hp)) return 0;
  return (size_t)hp.sz.total_bytes;
}

size_t msda_bwd_dev_workspace_bytes(const msda_desc* d) {
  g_err[0] = 0;
  if (validate(d)) return 0;
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  if (units == 0 || d->num_levels == 0 || d->num_points == 0) return 0;
  BwdHostPlan hp;
  const void* none[1] = {nullptr};
  if (plan_bwd(d, nullptr, none, 0, &hp)) return 0;
  return (size_t)hp.sz.total_bytes;
}

int msda_bwd(const msda_desc* d, const int32_t* host_spatial_shapes, const void* value,
             const void* sampling_locations, const void* attention_weights,
             const void* grad_output, void* grad_value, void* grad_sampling_locations,
             void* grad_attention_weights, void* workspace, size_t workspace_bytes,
             void* stream) {
  g_err[0] = 0;
  if (d && d->num_levels > 0 && !host_spatial_shapes && validate(d) == MSDA_OK)
    return fail(MSDA_ERR_INVALID, "host spatial shapes are NULL");
  return bwd_impl(d, host_spatial_shapes, nullptr, value, sampling_locations, attention_weights,
                  grad_output, grad_value, grad_sampling_locations, grad_attention_weights,
                  workspace, workspace_bytes, stream, "msda_bwd");
}

int msda_bwd_dev(const msda_desc* d, const int32_t* spatial_shapes, const void* value,
                 const void* sampling_locations, const void* attention_weights,
                 const void* grad_output, void* grad_value, void* grad_sampling_locations,
                 void* grad_attention_weights, void* workspace, size_t workspace_bytes,
                 void* stream) {
  g_err[0] = 0;
  return bwd_impl(d, nullptr, spatial_shapes, value, sampling_locations, attention_weights,
                  grad_output, grad_value, grad_sampling_locations, grad_attention_weights,
                  workspace, workspace_bytes, stream, "msda_bwd_dev");
}

size_t msda_bwd_fused_workspace_bytes(const msda_desc* d, const int32_t* host_spatial_shapes) {
  g_err[0] = 0;
  if (validate(d)) return 0;
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  if (units == 0 || d->num_levels == 0 || d->num_points == 0) return 0;
  if (!host_spatial_shapes) return fail(MSDA_ERR_INVALID, "host spatial shapes are NULL"), 0;
  FusedWs w;
  if (!fused_ws(d, host_spatial_shapes, &w)) return 0;
  return (size_t)w.total;
}

size_t msda_bwd_fused_dev_workspace_bytes(const msda_desc* d) {
  g_err[0] = 0;
  if (validate(d)) return 0;
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  if (units == 0 || d->num_levels == 0 || d->num_points == 0) return 0;
  FusedWs w;
  if (!fused_ws(d, nullptr, &w)) return 0;
  return (size_t)w.total;
}

int msda_bwd_fused(const msda_desc* d, const int32_t* host_spatial_shapes, const void* value,
                   const float* reference_points, const void* sampling_offsets,
                   const void* attention_logits, const void* grad_output, void* grad_value,
                   float* grad_reference_points, void* grad_sampling_offsets,
                   void* grad_attention_logits, void* workspace, size_t workspace_bytes,
                   void* stream) {
  g_err[0] = 0;
  if (d && d->num_levels > 0 && !host_spatial_shapes && validate(d) == MSDA_OK)
    return fail(MSDA_ERR_INVALID, "host spatial shapes are NULL");
  return fused_bwd_impl(d, host_spatial_shapes, nullptr, value, reference_points,
                        sampling_offsets, attention_logits, grad_output, grad_value,
                        grad_reference_points, grad_sampling_offsets, grad_attention_logits,
                        workspace, workspace_bytes, stream, "msda_bwd_fused");
}

int msda_bwd_fused_dev(const msda_desc* d, const int32_t* spatial_shapes, const void* value,
                       const float* reference_points, const void* sampling_offsets,
                       const void* attention_logits, const void* grad_output, void* grad_value,
                       float* grad_reference_points, void* grad_sampling_offsets,
                       void* grad_attention_logits, void* workspace, size_t workspace_bytes,
                       void* stream) {
  g_err[0] = 0;
  return fused_bwd_impl(d, nullptr, spatial_shapes, value, reference_points, sampling_offsets,
                        attention_logits, grad_output, grad_value, grad_reference_points,
                        grad_sampling_offsets, grad_attention_logits, workspace,
                        workspace_bytes, stream, "msda_bwd_fused_dev");
}

}  // extern "C"
