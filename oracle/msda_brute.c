/*
 * msda_brute.c — TEST INFRASTRUCTURE ONLY. Brute-force CPU restatement of multi-scale
 * deformable attention (forward and analytic backward), used as a checker by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg. Nothing in the msda_triton
 * package links or calls this file.
 *
 * It restates the reference's oracle msda2d_pytorch / msda3d_pytorch
 * (src/msda_triton/pytorch/msda_2d.py:58-114, src/msda_triton/pytorch/msda_3d.py:58-118),
 * i.e. per level: grid = 2*loc - 1, optional clamp to [-1+eps, 1-eps]
 * (msda_2d.py:66-68), F.grid_sample(bilinear, zeros, align_corners=False)
 * (msda_2d.py:92-98), times attention weight, summed over points and levels
 * (msda_2d.py:102-110) — as explicit loops over (b, q, h, l, p, corner, c) that call no
 * library sampling routine. The pixel coordinate is ((g+1)*size-1)/2 (ATen
 * GridSampler.h grid_sampler_unnormalize, align_corners=False); corners outside the
 * level contribute zero. Gradients follow the chain rule through the same steps:
 * d/dloc = 2 * (size/2) * d/du, masked to zero where the grid clamp was active
 * (backward of torch.clamp passes gradient for lo <= g <= hi).
 *
 * All sums are in double. coord_f32 = 1 computes the grid and pixel coordinate in float
 * with each operation rounded separately (the order ATen and the HIP kernels use), so
 * the selected corner matches an fp32 implementation exactly; coord_f32 = 0 computes
 * them in double.
 *
 * Layouts (contiguous): value (B,K,H,C); shapes (L,dim) as (H,W) or (D,H,W);
 * loc (B,Q,H,L,P,dim) with coordinate order (x,y[,z]); attn (B,Q,H,L,P); out (B,Q,H*C).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

typedef struct {
  double e, f;   /* weights of lower / upper corner */
  long i0;       /* lower corner index */
  int pass;      /* gradient passes the clamp */
  double u;      /* pixel coordinate */
} axis_t;

static axis_t make_axis(double loc, long size, int clamp, double eps, int coord_f32) {
  axis_t a;
  if (coord_f32) {
    volatile float g = 2.0f * (float)loc;
    g = g - 1.0f;
    const float lo = (float)(-1.0 + eps), hi = (float)(1.0 - eps);
    a.pass = !clamp || (g >= lo && g <= hi);
    if (clamp) g = g < lo ? lo : (g > hi ? hi : g);
    volatile float t = g + 1.0f;
    t = t * (float)size;
    t = t - 1.0f;
    t = t * 0.5f;
    const float u = t;
    const float u0 = floorf(u);
    volatile float f = u - u0;
    volatile float e = (u0 + 1.0f) - u;
    a.f = f;
    a.e = e;
    a.i0 = (long)u0;
    a.u = u;
  } else {
    double g = 2.0 * loc - 1.0;
    const double lo = -1.0 + eps, hi = 1.0 - eps;
    a.pass = !clamp || (g >= lo && g <= hi);
    if (clamp) g = g < lo ? lo : (g > hi ? hi : g);
    const double u = ((g + 1.0) * (double)size - 1.0) / 2.0;
    const double u0 = floor(u);
    a.f = u - u0;
    a.e = (u0 + 1.0) - u;
    a.i0 = (long)u0;
    a.u = u;
  }
  return a;
}

static int inside(long i, long n) { return i >= 0 && i < n; }

/* Shared traversal: for every sample, visit its 2^dim corners. */
typedef struct {
  int dim, B, H, C, Q, L, P;
  long K;
  const int64_t* shapes;
  int clamp;
  double eps;
  int coord_f32;
} prob_t;

static void level_geom(const prob_t* pr, int l, long* D, long* Hh, long* W, long* start) {
  long s = 0;
  for (int i = 0; i < l; ++i) {
    long n = 1;
    for (int k = 0; k < pr->dim; ++k) n *= (long)pr->shapes[i * pr->dim + k];
    s += n;
  }
  *start = s;
  if (pr->dim == 2) {
    *D = 1;
    *Hh = (long)pr->shapes[l * 2 + 0];
    *W = (long)pr->shapes[l * 2 + 1];
  } else {
    *D = (long)pr->shapes[l * 3 + 0];
    *Hh = (long)pr->shapes[l * 3 + 1];
    *W = (long)pr->shapes[l * 3 + 2];
  }
}

void msda_brute_fwd(int dim, int B, long K, int H, int C, int Q, int L, int P,
                    const int64_t* shapes, const double* value, const double* loc,
                    const double* attn, int clamp_grid, double clamp_eps, int coord_f32,
                    double* out) {
  prob_t pr = {dim, B, H, C, Q, L, P, K, shapes, clamp_grid, clamp_eps, coord_f32};
  const int nc = 1 << dim;
  memset(out, 0, sizeof(double) * (size_t)B * Q * H * C);
  for (int b = 0; b < B; ++b)
    for (int q = 0; q < Q; ++q)
      for (int h = 0; h < H; ++h) {
        double* o = out + (((size_t)b * Q + q) * H + h) * C;
        for (int l = 0; l < L; ++l) {
          long D, Hh, W, start;
          level_geom(&pr, l, &D, &Hh, &W, &start);
          for (int p = 0; p < P; ++p) {
            const size_t si = ((((size_t)b * Q + q) * H + h) * L + l) * P + p;
            const double a = attn[si];
            const double* lp = loc + si * dim;
            axis_t ax = make_axis(lp[0], W, clamp_grid, clamp_eps, coord_f32);
            axis_t ay = make_axis(lp[1], Hh, clamp_grid, clamp_eps, coord_f32);
            axis_t az = {1.0, 0.0, 0, 1, 0.0};
            if (dim == 3) az = make_axis(lp[2], D, clamp_grid, clamp_eps, coord_f32);
            for (int c = 0; c < nc; ++c) {
              const long x = ax.i0 + (c & 1), y = ay.i0 + ((c >> 1) & 1);
              const long z = dim == 3 ? az.i0 + ((c >> 2) & 1) : 0;
              if (!inside(x, W) || !inside(y, Hh) || !inside(z, D)) continue;
              double w = ((c & 1) ? ax.f : ax.e) * (((c >> 1) & 1) ? ay.f : ay.e);
              if (dim == 3) w *= ((c >> 2) & 1) ? az.f : az.e;
              const long k = start + (z * Hh + y) * W + x;
              const double* v = value + (((size_t)b * K + k) * H + h) * C;
              for (int ch = 0; ch < C; ++ch) o[ch] += a * w * v[ch];
            }
          }
        }
      }
}

void msda_brute_bwd(int dim, int B, long K, int H, int C, int Q, int L, int P,
                    const int64_t* shapes, const double* value, const double* loc,
                    const double* attn, int clamp_grid, double clamp_eps, int coord_f32,
                    const double* grad_out, double* grad_value, double* grad_loc,
                    double* grad_attn) {
  prob_t pr = {dim, B, H, C, Q, L, P, K, shapes, clamp_grid, clamp_eps, coord_f32};
  const int nc = 1 << dim;
  memset(grad_value, 0, sizeof(double) * (size_t)B * K * H * C);
  for (int b = 0; b < B; ++b)
    for (int q = 0; q < Q; ++q)
      for (int h = 0; h < H; ++h) {
        const double* g = grad_out + (((size_t)b * Q + q) * H + h) * C;
        for (int l = 0; l < L; ++l) {
          long D, Hh, W, start;
          level_geom(&pr, l, &D, &Hh, &W, &start);
          for (int p = 0; p < P; ++p) {
            const size_t si = ((((size_t)b * Q + q) * H + h) * L + l) * P + p;
            const double a = attn[si];
            const double* lp = loc + si * dim;
            axis_t ax = make_axis(lp[0], W, clamp_grid, clamp_eps, coord_f32);
            axis_t ay = make_axis(lp[1], Hh, clamp_grid, clamp_eps, coord_f32);
            axis_t az = {1.0, 0.0, 0, 1, 0.0};
            if (dim == 3) az = make_axis(lp[2], D, clamp_grid, clamp_eps, coord_f32);
            double s_attn = 0.0, du[3] = {0.0, 0.0, 0.0};
            for (int c = 0; c < nc; ++c) {
              const int cx = c & 1, cy = (c >> 1) & 1, cz = (c >> 2) & 1;
              const long x = ax.i0 + cx, y = ay.i0 + cy, z = dim == 3 ? az.i0 + cz : 0;
              if (!inside(x, W) || !inside(y, Hh) || !inside(z, D)) continue;
              const double wx = cx ? ax.f : ax.e, wy = cy ? ay.f : ay.e;
              const double wz = dim == 3 ? (cz ? az.f : az.e) : 1.0;
              const double sx = cx ? 1.0 : -1.0, sy = cy ? 1.0 : -1.0, sz = cz ? 1.0 : -1.0;
              const long k = start + (z * Hh + y) * W + x;
              const size_t vi = (((size_t)b * K + k) * H + h) * C;
              double dot = 0.0;
              for (int ch = 0; ch < C; ++ch) {
                dot += g[ch] * value[vi + ch];
                grad_value[vi + ch] += a * wx * wy * wz * g[ch];
              }
              s_attn += wx * wy * wz * dot;
              du[0] += sx * wy * wz * dot;
              du[1] += wx * sy * wz * dot;
              du[2] += wx * wy * sz * dot;
            }
            grad_attn[si] = s_attn;
            /* u = ((g+1)*size-1)/2, g = 2*loc-1  =>  du/dloc = size */
            grad_loc[si * dim + 0] = ax.pass ? a * du[0] * (double)W : 0.0;
            grad_loc[si * dim + 1] = ay.pass ? a * du[1] * (double)Hh : 0.0;
            if (dim == 3) grad_loc[si * dim + 2] = az.pass ? a * du[2] * (double)D : 0.0;
          }
        }
      }
}

/* Pixel coordinates u of every (sample, axis), in the loc layout; used by tests to find
   samples whose coordinate lies within a tolerance of a cell edge. */
void msda_brute_coords(int dim, int B, int H, int Q, int L, int P, const int64_t* shapes,
                       const double* loc, int clamp_grid, double clamp_eps, int coord_f32,
                       double* u_out) {
  prob_t pr = {dim, B, H, 0, Q, L, P, 0, shapes, clamp_grid, clamp_eps, coord_f32};
  for (int b = 0; b < B; ++b)
    for (int q = 0; q < Q; ++q)
      for (int h = 0; h < H; ++h)
        for (int l = 0; l < L; ++l) {
          long D, Hh, W, start;
          level_geom(&pr, l, &D, &Hh, &W, &start);
          const long sz[3] = {W, Hh, D};
          for (int p = 0; p < P; ++p) {
            const size_t si = ((((size_t)b * Q + q) * H + h) * L + l) * P + p;
            for (int k = 0; k < dim; ++k)
              u_out[si * dim + k] =
                  make_axis(loc[si * dim + k], sz[k], clamp_grid, clamp_eps, coord_f32).u;
          }
        }
}
