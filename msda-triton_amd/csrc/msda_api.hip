// msda_api.hip — extern "C" entry points declared in include/msda.h.
//
// Host-side work per call: validate the descriptor, pick the kernel instantiation,
// split the batch into launches whose byte offsets fit the 32-bit buffer addressing
// the kernels use, and enqueue everything on the caller's stream. No allocation,
// no synchronisation, no global mutable state except the thread-local error text.
#include <math.h>
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

// Lanes per unit and vector width for C channels of `vb` bytes each.
struct Layout {
  int vec_bytes;  // bytes per lane per row
  int nvec;       // C / VEC
  int lpu_log2;   // lanes per unit = 2^lpu_log2
  int hg_log2;    // heads per 128-byte line group
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
  // Heads whose rows share a 128-byte line are kept on the same lanes' neighbourhood.
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
    return fail(MSDA_ERR_INVALID,
                "invalid sizes: B=%d K=%lld H=%d C=%d Q=%lld L=%d P=%d", d->batch,
                (long long)d->num_keys, d->num_heads, d->channels, (long long)d->num_queries,
                d->num_levels, d->num_points);
  if (d->value_dtype < MSDA_F32 || d->value_dtype > MSDA_BF16)
    return fail(MSDA_ERR_DTYPE, "value dtype code %d is not fp32, fp16 or bf16", d->value_dtype);
  if (d->coord_dtype != d->value_dtype && d->coord_dtype != MSDA_F32)
    return fail(MSDA_ERR_DTYPE,
                "sampling_locations/attention_weights dtype %s must equal value dtype %s or be "
                "float32",
                dtype_name(d->coord_dtype), dtype_name(d->value_dtype));
  if (d->reserved != 0) return fail(MSDA_ERR_INVALID, "reserved field must be 0");
  if (!isfinite(d->clamp_eps)) return fail(MSDA_ERR_INVALID, "clamp_eps must be finite");
  if (d->num_keys > (int64_t)kLim31)
    return fail(MSDA_ERR_INVALID, "number of keys (%lld) exceeds int32 range",
                (long long)d->num_keys);
  if (d->num_levels > msda::kMaxLevels)
    return fail(MSDA_ERR_INVALID, "at most %d levels are supported, got %d", msda::kMaxLevels,
                d->num_levels);
  const uint64_t lpd = (uint64_t)d->num_levels * d->num_points * d->dim;
  if (lpd > (uint64_t)1 << 24)
    return fail(MSDA_ERR_INVALID, "levels*points too large (%llu)", (unsigned long long)lpd);
  // One batch must fit a launch: value bytes (and fp32 accumulator bytes) and
  // lanes of one batch below 2^31.
  const uint64_t per_b_acc = (uint64_t)d->num_keys * d->num_heads * d->channels * 4ull;
  if (per_b_acc > kLim31)
    return fail(MSDA_ERR_INVALID,
                "value slice of one batch is too large: K*H*C*4 = %llu bytes exceeds 2^31-1",
                (unsigned long long)per_b_acc);
  const uint64_t per_b_lanes = (uint64_t)d->num_queries * d->num_heads * 64ull;
  if (per_b_lanes > kLim31)
    return fail(MSDA_ERR_INVALID, "Q*H of one batch too large (%llu units)",
                (unsigned long long)((uint64_t)d->num_queries * d->num_heads));
  return MSDA_OK;
}

// Batches per launch such that every 32-bit in-kernel offset stays below 2^31.
int64_t batches_per_launch(const msda_desc* d, const Layout& lay) {
  const uint64_t per_b_acc = (uint64_t)d->num_keys * d->num_heads * d->channels * 4ull;
  const uint64_t per_b_lanes = ((uint64_t)d->num_queries * d->num_heads) << lay.lpu_log2;
  uint64_t nb = (uint64_t)d->batch;
  if (per_b_acc) nb = nb < kLim31 / per_b_acc ? nb : kLim31 / per_b_acc;
  if (per_b_lanes) nb = nb < kLim31 / per_b_lanes ? nb : kLim31 / per_b_lanes;
  return nb < 1 ? 1 : (int64_t)nb;
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
  const uint64_t vb = (uint64_t)d->num_keys * H * d->channels;
  p->value_bytes = (uint32_t)(nb * vb * elem_bytes(d->value_dtype));
  p->acc_bytes = (uint32_t)(nb * vb * 4ull);
}

}  // namespace

extern "C" {

int msda_abi_version(void) { return MSDA_ABI_VERSION; }

const char* msda_last_error(void) { return g_err; }

int msda_validate(const msda_desc* desc) {
  g_err[0] = 0;
  return validate(desc);
}

int msda_fwd(const msda_desc* d, const void* value, const int32_t* spatial_shapes,
             const int32_t* level_start, const void* sampling_locations,
             const void* attention_weights, void* output, void* stream) {
  g_err[0] = 0;
  int rc = validate(d);
  if (rc) return rc;
  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  if (units == 0) return MSDA_OK;
  const bool has_samples = d->num_levels > 0 && d->num_points > 0;
  if (!output || (d->num_keys > 0 && !value) ||
      (has_samples && (!sampling_locations || !attention_weights)) ||
      (d->num_levels > 0 && (!spatial_shapes || !level_start)))
    return fail(MSDA_ERR_INVALID, "msda_fwd: required pointer is NULL");
  const void* vptrs[2] = {value, output};
  Layout lay;
  if ((rc = choose_layout(d, vptrs, 2, &lay))) return rc;
  msda::LaunchFn fn = msda::get_fwd_launcher(d->dim, d->value_dtype, d->coord_dtype, lay.vec_bytes);
  if (!fn) return fail(MSDA_ERR_DTYPE, "no forward kernel for this dtype combination");

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
    hipError_t e = fn(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(MSDA_ERR_HIP, "msda_fwd launch failed: %s", hipGetErrorString(e));
  }
  return MSDA_OK;
}

size_t msda_bwd_workspace_bytes(const msda_desc* d) {
  if (!d || d->value_dtype == MSDA_F32) return 0;
  if (d->batch <= 0 || d->num_keys <= 0) return 0;
  return (size_t)d->batch * (size_t)d->num_keys * (size_t)d->num_heads * (size_t)d->channels * 4u;
}

int msda_bwd(const msda_desc* d, const void* value, const int32_t* spatial_shapes,
             const int32_t* level_start, const void* sampling_locations,
             const void* attention_weights, const void* grad_output, void* grad_value,
             void* grad_sampling_locations, void* grad_attention_weights, void* workspace,
             size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = validate(d);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t nval = (size_t)d->batch * (size_t)d->num_keys * d->num_heads * d->channels;
  const size_t need = msda_bwd_workspace_bytes(d);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MSDA_ERR_WORKSPACE, "msda_bwd needs %zu workspace bytes, got %zu", need,
                workspace_bytes);
  if (nval && !grad_value) return fail(MSDA_ERR_INVALID, "msda_bwd: grad_value is NULL");
  if (need && ((uintptr_t)workspace % 16) != 0)
    return fail(MSDA_ERR_INVALID, "msda_bwd: workspace must be 16-byte aligned");
  float* acc = d->value_dtype == MSDA_F32 ? static_cast<float*>(grad_value)
                                          : static_cast<float*>(workspace);
  hipError_t e = msda::launch_fill_zero(acc, nval, st);
  if (e != hipSuccess) return fail(MSDA_ERR_HIP, "msda_bwd clear failed: %s", hipGetErrorString(e));

  const uint64_t units = (uint64_t)d->batch * d->num_queries * d->num_heads;
  const bool has_samples = d->num_levels > 0 && d->num_points > 0;
  if (units > 0 && has_samples) {
    if ((d->num_keys > 0 && !value) || !sampling_locations || !attention_weights || !grad_output ||
        !grad_sampling_locations || !grad_attention_weights || !spatial_shapes || !level_start)
      return fail(MSDA_ERR_INVALID, "msda_bwd: required pointer is NULL");
    const void* vptrs[2] = {value, grad_output};
    Layout lay;
    if ((rc = choose_layout(d, vptrs, 2, &lay))) return rc;
    msda::LaunchFn fn =
        msda::get_bwd_launcher(d->dim, d->value_dtype, d->coord_dtype, lay.vec_bytes);
    if (!fn) return fail(MSDA_ERR_DTYPE, "no backward kernel for this dtype combination");
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
      p.grad_out = static_cast<const char*>(grad_output) + (uint64_t)b0 * qh * d->channels * sv;
      p.grad_acc = acc + (uint64_t)b0 * kv;
      p.grad_loc = static_cast<char*>(grad_sampling_locations) + (uint64_t)b0 * qh * LP * d->dim * sc;
      p.grad_attn = static_cast<char*>(grad_attention_weights) + (uint64_t)b0 * qh * LP * sc;
      p.shapes = spatial_shapes;
      p.starts = level_start;
      e = fn(p, st);
      if (e != hipSuccess)
        return fail(MSDA_ERR_HIP, "msda_bwd launch failed: %s", hipGetErrorString(e));
    }
  }
  if (d->value_dtype != MSDA_F32) {
    e = msda::launch_narrow(acc, grad_value, d->value_dtype, nval, st);
    if (e != hipSuccess)
      return fail(MSDA_ERR_HIP, "msda_bwd narrow failed: %s", hipGetErrorString(e));
  }
  return MSDA_OK;
}

}  // extern "C"
