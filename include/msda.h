/*
 * msda.h — C ABI of the MI355X (gfx950) multi-scale deformable attention library.
 *
 * One shared library, libmsda_hip.so, exports these entry points. They take plain
 * device pointers, sizes and a hipStream_t passed as void*; no torch or HIP types
 * appear in the signatures, so any FFI (ctypes, cffi, pybind11, a C++ caller) can bind
 * them. The Python package msda_triton binds them through ctypes.
 *
 * Tensor contract (identical to msda_triton's, reference README.md:60-68):
 *   value               (B, K, H, C)        value_dtype, contiguous
 *   spatial_shapes      (L, dim)  int32     rows are (H_l, W_l) for dim 2 and
 *                                           (D_l, H_l, W_l) for dim 3; device memory for
 *                                           msda_fwd and msda_bwd_dev, host memory for
 *                                           msda_bwd and msda_bwd_fused
 *   level_start         (L,)      int32     device memory (msda_fwd); exclusive prefix
 *                                           sum of the per-level sizes (row-major
 *                                           flattening of K)
 *   sampling_locations  (B, Q, H, L, P, dim) coord_dtype, contiguous, order (x, y[, z])
 *                                           with x along W, y along H, z along D
 *   attention_weights   (B, Q, H, L, P)      coord_dtype, contiguous
 *   output              (B, Q, H*C)          value_dtype, contiguous
 *
 * Every call returns an msda_status. On failure, msda_last_error() returns a
 * thread-local message that names the failing check. Calls enqueue work on `stream`
 * and do not synchronise. Calls on different streams or threads are independent:
 * the library holds no mutable global state apart from the thread-local error text.
 */
#ifndef MSDA_H_
#define MSDA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSDA_ABI_VERSION 5

typedef enum msda_dtype {
  MSDA_F32 = 0,
  MSDA_F16 = 1,
  MSDA_BF16 = 2
} msda_dtype;

typedef enum msda_status {
  MSDA_OK = 0,
  MSDA_ERR_INVALID = 1,         /* a size, pointer or flag is out of range */
  MSDA_ERR_DTYPE = 2,           /* unsupported dtype or dtype combination */
  MSDA_ERR_WORKSPACE = 3,       /* workspace missing or too small */
  MSDA_ERR_HIP = 4              /* a HIP runtime call failed (launch error) */
} msda_status;

/* Problem descriptor shared by forward and backward. All counts are element counts. */
typedef struct msda_desc {
  int32_t dim;          /* 2: bilinear over (H, W); 3: trilinear over (D, H, W) */
  int32_t batch;        /* B */
  int64_t num_keys;     /* K = sum over levels of prod(shape_l) */
  int32_t num_heads;    /* H */
  int32_t channels;     /* C, channels per head */
  int64_t num_queries;  /* Q */
  int32_t num_levels;   /* L */
  int32_t num_points;   /* P */
  int32_t value_dtype;  /* msda_dtype of value, output, grad_output and grad_value */
  int32_t coord_dtype;  /* msda_dtype of sampling_locations, attention_weights and their
                           gradients; must equal value_dtype or be MSDA_F32 */
  int32_t clamp_grid;   /* nonzero: clamp the [-1, 1] sampling grid to [-1+eps, 1-eps] */
  int32_t flags;        /* MSDA_FLAG_* bits; 0 for none */
  double clamp_eps;     /* eps of the clamp above (reference default 1e-4) */
} msda_desc;

/*
 * msda_desc.flags bit, for the backward entry points only (msda_bwd, msda_bwd_dev,
 * msda_bwd_fused, msda_bwd_fused_dev, msda_bwd_noalloc; the forward entry points and their
 * workspace queries reject it): `value` points to a head-major (B, H, K, C) copy of the
 * value tensor instead of the (B, K, H, C) tensor itself, such as the copy msda_fwd leaves
 * at the start of its workspace when msda_fwd_workspace_bytes() equals the whole value's
 * bytes. The backward then reads value rows in that layout (it never copies value, so the
 * flag only spares the caller from keeping the original tensor). The caller keeps the copy
 * alive and unchanged until the backward has run. No counterpart in the reference.
 */
#define MSDA_FLAG_VALUE_HEAD_MAJOR 1

/* ABI version of the loaded library (MSDA_ABI_VERSION it was built with). */
int msda_abi_version(void);

/* Thread-local text of the last error raised on this thread ("" if none). */
const char* msda_last_error(void);

/*
 * Host-only validation of a descriptor: sizes, dtypes and 32-bit index limits.
 * Touches no device. msda_fwd and msda_bwd run the same checks first.
 */
int msda_validate(const msda_desc* desc);

/*
 * Bytes of optional device workspace that lets msda_fwd gather from a head-major copy of
 * value (B, H, K, C): returned when value rows are shorter than a 128-byte line, there is
 * more than one head, the keys' line footprint exceeds one XCD's 4 MB L2 and the gathers
 * outnumber the keys at least eightfold (e.g. 76.7 MB for the 3D 4-level workload), else 0.
 * No counterpart in the reference, whose kernels always read the (B, K, H, C) layout.
 */
size_t msda_fwd_workspace_bytes(const msda_desc* desc);

/*
 * Forward: output = sum_l sum_p attn[b,q,h,l,p] * sample(value[b, level l, h, :], loc[b,q,h,l,p])
 * with bilinear (dim 2) or trilinear (dim 3) sampling, zero padding outside the level,
 * align_corners=False, fp32 accumulation, and output rounded once to value_dtype.
 *
 * `workspace` is optional: with at least msda_fwd_workspace_bytes() bytes (aligned to 16
 * bytes) the call first copies value into it in head-major order and gathers from the
 * copy; with NULL or fewer bytes it gathers from value directly. The output is the same
 * either way, bit for bit.
 *
 * Replaces the reference's _fwd_kernel_2d launch and permute/cast epilogue
 * (src/msda_triton/triton/msda_2d.py:606-651) and the 3D equivalent
 * (src/msda_triton/triton/msda_3d.py:749-794).
 */
int msda_fwd(const msda_desc* desc,
             const void* value,
             const int32_t* spatial_shapes,
             const int32_t* level_start,
             const void* sampling_locations,
             const void* attention_weights,
             void* output,
             void* workspace,
             size_t workspace_bytes,
             void* stream);

/*
 * Bytes of device workspace msda_bwd needs for this descriptor and these level shapes
 * (0 when there is nothing to sample; it includes the head-major value copy described at
 * msda_fwd_workspace_bytes when that applies). host_spatial_shapes is a HOST array of L*dim int32
 * laid out like spatial_shapes; the backward plans its spatial tiling from it. Returns 0
 * and sets msda_last_error() if the descriptor or shapes are invalid.
 */
size_t msda_bwd_workspace_bytes(const msda_desc* desc, const int32_t* host_spatial_shapes);

/*
 * Backward of msda_fwd with respect to value, sampling_locations and attention_weights.
 *
 * grad_value, grad_sampling_locations and grad_attention_weights are fully overwritten
 * (each element exactly once, with plain stores), in the dtypes of their inputs.
 * Gradients of clamped grid coordinates are zero, matching the backward of torch.clamp.
 * grad_value is accumulated in fp32 in on-chip memory per spatial tile, so no device-wide
 * atomics are used; the order of the fp32 additions within a tile is not fixed, so its
 * low-order bits may vary between runs. Levels with more than 8192 tiles per head in total
 * (about 1 M cells) are accumulated instead with global fp32 atomics into an fp32 copy of
 * grad_value in the workspace, then rounded once. `workspace` must hold
 * msda_bwd_workspace_bytes() bytes, 256-byte aligned; it needs no initialisation.
 *
 * Replaces the reference's MSDA2DFn.backward body (src/msda_triton/triton/msda_2d.py:778-853,
 * kernel _bwd_kernel_2d :263-510) and MSDA3DFn.backward (src/msda_triton/triton/msda_3d.py:
 * 920-996, kernel _bwd_kernel :291-653).
 */
int msda_bwd(const msda_desc* desc,
             const int32_t* host_spatial_shapes,
             const void* value,
             const void* sampling_locations,
             const void* attention_weights,
             const void* grad_output,
             void* grad_value,
             void* grad_sampling_locations,
             void* grad_attention_weights,
             void* workspace,
             size_t workspace_bytes,
             void* stream);

/*
 * Bytes of device workspace msda_bwd_dev needs for this descriptor (0 when there is nothing
 * to sample), sized without the level shapes: from K it estimates the spatial tiles the
 * backward bins samples into, and it adds an fp32 copy of grad_value for the atomic path the
 * kernels fall back to on the device when the levels need more tiles than estimated (levels
 * that are thin along an axis). Returns 0 and sets msda_last_error() if the descriptor is
 * invalid.
 */
size_t msda_bwd_dev_workspace_bytes(const msda_desc* desc);

/*
 * msda_bwd with the level shapes in DEVICE memory (spatial_shapes as for msda_fwd). The
 * host never reads them: the first kernel derives the tile geometry from them on the
 * device, so the call neither copies the shapes to the host nor synchronises, and the
 * whole sequence can be captured in a HIP graph. Results are those of msda_bwd on the same
 * shapes, bit for bit in grad_sampling_locations and grad_attention_weights, and with the
 * same fp32 accumulation of grad_value. If the shapes disagree with K (sum of the level
 * sizes), every gradient is filled with NaN, since the error can no longer be returned.
 * `workspace` must hold msda_bwd_dev_workspace_bytes() bytes, 256-byte aligned.
 *
 * Replaces the reference's backward for GPU-resident shapes, which reads the device level
 * tables saved by the forward (src/msda_triton/triton/msda_2d.py:76-82, :799-851;
 * src/msda_triton/triton/msda_3d.py:71-77, :942-996).
 */
int msda_bwd_dev(const msda_desc* desc,
                 const int32_t* spatial_shapes,
                 const void* value,
                 const void* sampling_locations,
                 const void* attention_weights,
                 const void* grad_output,
                 void* grad_value,
                 void* grad_sampling_locations,
                 void* grad_attention_weights,
                 void* workspace,
                 size_t workspace_bytes,
                 void* stream);

/*
 * Fused producer variant of msda_fwd: instead of sampling_locations and attention_weights
 * it reads what the attention modules produce before them, and forms both in fp32 inside
 * the kernel:
 *   loc[b,q,h,l,p,d] = reference_points[b,q,l,d] + sampling_offsets[b,q,h,l,p,d] / size_l[d]
 *                      with size_l = (W_l, H_l) for dim 2 and (W_l, H_l, D_l) for dim 3
 *   attn[b,q,h,l,p]  = softmax over (l, p) of attention_logits[b,q,h,:]
 *   reference_points  (B, Q, L, dim)        float32, contiguous, in [0, 1] per level
 *   sampling_offsets  (B, Q, H, L, P, dim)  coord_dtype, contiguous, in pixels of level l
 *   attention_logits  (B, Q, H, L, P)       coord_dtype, contiguous
 * Other arguments, the workspace and the output are as for msda_fwd. The locations and
 * weights never reach memory.
 *
 * Replaces the location and weight formation of the reference modules followed by the
 * forward launch: src/msda_triton/pytorch/msda_2d.py:303-339 (offset normaliser, softmax
 * over L*P, reference + offset / normaliser) and src/msda_triton/pytorch/msda_3d.py:314-350,
 * then src/msda_triton/triton/msda_2d.py:606-651 / msda_3d.py:749-794.
 */
int msda_fwd_fused(const msda_desc* desc,
                   const void* value,
                   const int32_t* spatial_shapes,
                   const int32_t* level_start,
                   const float* reference_points,
                   const void* sampling_offsets,
                   const void* attention_logits,
                   void* output,
                   void* workspace,
                   size_t workspace_bytes,
                   void* stream);

/*
 * Bytes of device workspace msda_bwd_fused needs (0 when there is nothing to sample): fp32
 * locations, weights and their gradients, plus the msda_bwd workspace for them.
 */
size_t msda_bwd_fused_workspace_bytes(const msda_desc* desc, const int32_t* host_spatial_shapes);

/*
 * Backward of msda_fwd_fused with respect to value, reference_points, sampling_offsets and
 * attention_logits:
 *   grad_sampling_offsets = grad_loc / size_l
 *   grad_reference_points = sum over (h, p) of grad_loc                       (float32)
 *   grad_attention_logits = attn * (grad_attn - sum over (l, p) of attn * grad_attn)
 * where grad_loc and grad_attn are msda_bwd's gradients at the fp32 locations and weights
 * the forward formed. All outputs are fully overwritten; grad_value as in msda_bwd.
 *
 * Replaces autograd through the same reference module lines as msda_fwd_fused plus the
 * MSDA2DFn / MSDA3DFn backward (src/msda_triton/triton/msda_2d.py:778-853,
 * msda_3d.py:920-996).
 */
int msda_bwd_fused(const msda_desc* desc,
                   const int32_t* host_spatial_shapes,
                   const void* value,
                   const float* reference_points,
                   const void* sampling_offsets,
                   const void* attention_logits,
                   const void* grad_output,
                   void* grad_value,
                   float* grad_reference_points,
                   void* grad_sampling_offsets,
                   void* grad_attention_logits,
                   void* workspace,
                   size_t workspace_bytes,
                   void* stream);

/* msda_bwd_fused_workspace_bytes for msda_bwd_fused_dev: sized without the level shapes, as
 * msda_bwd_dev_workspace_bytes is. */
size_t msda_bwd_fused_dev_workspace_bytes(const msda_desc* desc);

/*
 * msda_bwd_fused with the level shapes in DEVICE memory: the reciprocals of the level
 * extents are computed on the device (the fused forward's division, so the locations are
 * bit-identical) and the inner backward is msda_bwd_dev's. No host read of the shapes, no
 * synchronisation. Same outputs as msda_bwd_fused on the same shapes.
 *
 * Replaces autograd through the reference modules' location and weight formation
 * (src/msda_triton/pytorch/msda_2d.py:303-339, msda_3d.py:314-350) with GPU-resident
 * shapes, followed by the GPU-shapes backward (src/msda_triton/triton/msda_2d.py:76-82,
 * :799-851; msda_3d.py:71-77, :942-996).
 */
int msda_bwd_fused_dev(const msda_desc* desc,
                       const int32_t* spatial_shapes,
                       const void* value,
                       const float* reference_points,
                       const void* sampling_offsets,
                       const void* attention_logits,
                       const void* grad_output,
                       void* grad_value,
                       float* grad_reference_points,
                       void* grad_sampling_offsets,
                       void* grad_attention_logits,
                       void* workspace,
                       size_t workspace_bytes,
                       void* stream);

/* Bytes of the static device scratch msda_bwd_noalloc uses as its workspace (256 MiB per GPU). */
#define MSDA_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)

/*
 * msda_bwd that allocates nothing: no counterpart in the reference. It is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Arguments and results are those of msda_bwd, without
 * the workspace: the workspace is a static device array of MSDA_NOALLOC_SCRATCH_BYTES that
 * each GPU the library runs on holds from module load until the process ends, its device
 * address looked up once per device on the first call there. A problem whose
 * msda_bwd_workspace_bytes() exceeds that size is refused with MSDA_ERR_WORKSPACE (the
 * 2D encoder workload, B=2 Q=K=19947, needs about 165 MB; the 3D 4-level one, about
 * 600 MB, does not fit). Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams or threads) race, so callers serialise them.
 */
int msda_bwd_noalloc(const msda_desc* desc,
                     const int32_t* host_spatial_shapes,
                     const void* value,
                     const void* sampling_locations,
                     const void* attention_weights,
                     const void* grad_output,
                     void* grad_value,
                     void* grad_sampling_locations,
                     void* grad_attention_weights,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSDA_H_ */
