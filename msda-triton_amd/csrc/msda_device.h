// msda_device.h — device-side building blocks shared by the gfx950 MSDA kernels.
//
// Everything here is written for CDNA4 (gfx950, wave64): buffer-resource loads whose
// hardware range check turns out-of-level corners into zeros without a branch,
// 16-byte row loads, DPP / ds_swizzle lane exchanges, and fp32 accumulation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msda {

constexpr int kBlock = 256;            // threads per workgroup (4 waves)
constexpr int kWave = 64;
constexpr int kCusPerXcd = 32;         // gfx950 (MI350 / MI355): 32 compute units per XCD
constexpr uint32_t kOobOffset = 0x80000000u;  // buffer offset that always fails the range check

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------------------
// Division by a loop-invariant 32-bit divisor: q = (mulhi(n, m) + n) >> s, with the sum
// formed in 64 bits. Host side picks m and s (round-up method, Granlund & Montgomery 1994).
struct FastDiv {
  uint32_t d, m, s;
};

// Workgroup barrier that orders LDS only: waits for this wave's LDS operations, not for
// its outstanding global loads (which __syncthreads' workgroup fence also waits for), so
// loads issued before it stay in flight across it. For phases that share data through
// LDS alone.
__device__ inline void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__host__ __device__ inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t l = 0;
  while (l < 32 && (1ull << l) < d) ++l;
  f.s = l;
  f.m = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
  return f;
}

__device__ inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
  uint32_t t = __umulhi(n, f.m);
  return (uint32_t)(((uint64_t)t + n) >> f.s);
}

// ---------------------------------------------------------------------------------------
// Buffer resource over a byte range [base, base + nbytes). Loads whose offset is beyond
// nbytes return zero and stores / atomics there are dropped by the hardware.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes,
                                           0x00020000);
}

// ---------------------------------------------------------------------------------------
// Element types. Value rows are loaded as raw dwords and widened to fp32 in registers.
struct F32 {
  using T = float;
  static constexpr int kBytes = 4;
};
struct F16 {
  using T = _Float16;
  static constexpr int kBytes = 2;
};
struct BF16 {
  using T = __bf16;
  static constexpr int kBytes = 2;
};

// Raw storage for VEC elements of type E (VEC * bytes is 2, 4, 8 or 16).
template <int NBYTES>
struct RawVec;
template <>
struct RawVec<16> {
  u32x4 v;
};
template <>
struct RawVec<8> {
  u32x2 v;
};
template <>
struct RawVec<4> {
  uint32_t v;
};
template <>
struct RawVec<2> {
  uint16_t v;
};

template <int NBYTES>
__device__ inline RawVec<NBYTES> buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <>
__device__ inline RawVec<16> buf_load<16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return {__builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0)};
}
template <>
__device__ inline RawVec<8> buf_load<8>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return {__builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0)};
}
template <>
__device__ inline RawVec<4> buf_load<4>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return {__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0)};
}
template <>
__device__ inline RawVec<2> buf_load<2>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return {__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0)};
}

template <int NBYTES>
__device__ inline RawVec<NBYTES> glb_load(const void* p) {
  return *reinterpret_cast<const RawVec<NBYTES>*>(p);
}

// dword i (or the single 16-bit word) of a raw vector
template <int NBYTES>
__device__ inline uint32_t raw_dword(const RawVec<NBYTES>& r, int i) {
  if constexpr (NBYTES == 16) return r.v[i];
  else if constexpr (NBYTES == 8) return r.v[i];
  else if constexpr (NBYTES == 4) return r.v;
  else return (uint32_t)r.v;
}

// Reinterpret a 32-bit word as fp32 and back. The argument is taken by value: clang's
// __builtin_bit_cast applied directly to an element of an ext_vector_type value reads the
// vector's first element whatever the index, so vector elements must pass through these.
__device__ inline float as_float(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ inline uint32_t as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }

__device__ inline float bf16lo(uint32_t u) { return __builtin_bit_cast(float, u << 16); }
__device__ inline float bf16hi(uint32_t u) { return __builtin_bit_cast(float, u & 0xffff0000u); }
__device__ inline float f16lo(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
}
__device__ inline float f16hi(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}

// Widen VEC elements held in a raw vector into fp32 registers.
template <typename E, int VEC>
__device__ inline void widen(const RawVec<VEC * E::kBytes>& r, float (&o)[VEC]) {
  if constexpr (E::kBytes == 4) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = __builtin_bit_cast(float, raw_dword(r, i));
  } else if constexpr (VEC == 1) {
    uint32_t u = raw_dword(r, 0);
    if constexpr (sizeof(typename E::T) == 2 && __is_same(E, BF16)) o[0] = bf16lo(u);
    else o[0] = f16lo(u);
  } else {
#pragma unroll
    for (int i = 0; i < VEC / 2; ++i) {
      uint32_t u = raw_dword(r, i);
      if constexpr (__is_same(E, BF16)) {
        o[2 * i] = bf16lo(u);
        o[2 * i + 1] = bf16hi(u);
      } else {
        o[2 * i] = f16lo(u);
        o[2 * i + 1] = f16hi(u);
      }
    }
  }
}

// acc + a.lo * b.lo + a.hi * b.hi for two packed 16-bit pairs, in fp32. Both products of
// 16-bit floats are exact in fp32, so this equals two fp32 FMAs on the widened values up
// to the rounding of the sum.
template <typename E>
__device__ inline float dot2_acc(uint32_t a, uint32_t b, float acc) {
  if constexpr (__is_same(E, BF16)) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), acc,
                                           false);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), acc, false);
  }
}

// Two fp32 values packed into one dword of 16-bit elements (a in the low half), rounded to
// nearest even; exact for values that are representable in the 16-bit type.
template <typename E>
__device__ inline uint32_t pack2(float a, float b) {
  if constexpr (__is_same(E, BF16)) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// fp32 -> storage type, round to nearest even (hardware conversions on gfx950).
template <typename E>
__device__ inline typename E::T narrow(float x) {
  return (typename E::T)x;
}

template <typename E, int VEC>
__device__ inline void store_vec(typename E::T* p, const float (&a)[VEC]) {
  if constexpr (E::kBytes == 4) {
    if constexpr (VEC % 4 == 0) {
#pragma unroll
      for (int i = 0; i < VEC; i += 4)
        *reinterpret_cast<float4*>(p + i) = make_float4(a[i], a[i + 1], a[i + 2], a[i + 3]);
    } else if constexpr (VEC == 2) {
      *reinterpret_cast<float2*>(p) = make_float2(a[0], a[1]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) p[i] = a[i];
    }
  } else {
    typedef typename E::T T;
    typedef T tvec __attribute__((ext_vector_type(VEC)));
    tvec v;
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = narrow<E>(a[i]);
    *reinterpret_cast<tvec*>(p) = v;
  }
}

// Load one coordinate-type scalar as fp32.
template <typename E>
__device__ inline float ld_scalar(const typename E::T* p) {
  return (float)*p;
}

// ---------------------------------------------------------------------------------------
// Lane exchanges inside a group of 2^k lanes of one wave64.
__device__ inline float xor_lane(float v, int m) {
  int iv = __builtin_bit_cast(int, v);
  int r;
  switch (m) {
    case 1:  // quad_perm [1,0,3,2]
      r = __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, true);
      break;
    case 2:  // quad_perm [2,3,0,1]
      r = __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, true);
      break;
    case 4:
      r = __builtin_amdgcn_ds_swizzle(iv, 0x1F | (4 << 10));
      break;
    case 8:
      r = __builtin_amdgcn_ds_swizzle(iv, 0x1F | (8 << 10));
      break;
    case 16:
      r = __builtin_amdgcn_ds_swizzle(iv, 0x1F | (16 << 10));
      break;
    default:
      r = __shfl_xor(iv, m, kWave);
      break;
  }
  return __builtin_bit_cast(float, r);
}

// Sum over the 2^lg lanes of an aligned lane group; every lane receives the total.
__device__ inline float group_sum(float v, int lg) {
  for (int i = 0; i < lg; ++i) v += xor_lane(v, 1 << i);
  return v;
}

// ---------------------------------------------------------------------------------------
// Workgroup index with XCD-contiguous ownership: the hardware deals workgroups to the
// device's `xcds` XCDs round-robin (8 on a whole MI355X, fewer in a partition), so
// physical block i runs on XCD i % xcds. Remap so XCD x owns one contiguous range of
// logical blocks; consecutive logical blocks cover consecutive (batch, head-group) slices,
// which then stay resident in that XCD's L2.
__device__ inline uint32_t xcd_logical_block(uint32_t bid, uint32_t nblocks, uint32_t xcds) {
  uint32_t xcd = bid % xcds;
  uint32_t idx = bid / xcds;
  uint32_t per = nblocks / xcds;
  uint32_t rem = nblocks % xcds;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

}  // namespace msda
