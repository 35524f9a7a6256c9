// probes.hip — microbenchmarks behind the kernels' design choices on MI355X (gfx950).
// Measurement only: nothing in msda_triton links this library. benchmarks/probes.py builds
// it (libmsda_probes.so), runs every probe and prints the summary committed in profiles/.
//
//  * gather: random rows of R bytes (64 = a bf16 C=32 head row, 128 = a full line) read by
//    groups of R/16 lanes with one 16-byte load each, U independent rows in flight per
//    lane, from a table of S bytes (L2-, MALL- or HBM-resident by its size). Rows per
//    second are the line-request rate the forward and sample-gradient kernels depend on.
//  * atomics: groups of 32 lanes add 32 consecutive fp32 (or 64 packed-bf16) channels of a
//    random 128-byte row of a table, as a per-corner grad_value scatter would; element
//    additions per second.
//  * LDS: integer (ds_add_u32) against fp32 (ds_add_f32) atomics at random addresses of
//    a 64 KB array, and plain stores for comparison; lane operations per clock per CU.
//
// Every index is reduced modulo its table, so every access stays in bounds.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;

__device__ inline uint32_t hash32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// R-byte rows: lane j of each group of R/16 lanes loads bytes [16 j, 16 j + 16) of the row.
template <int R, int U>
__global__ __launch_bounds__(kThreads) void gather_probe(const char* __restrict__ table, uint32_t rows,
                                                        uint32_t iters, uint32_t* __restrict__ sink) {
  constexpr int G = R / 16;
  const uint32_t tid = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t grp = tid / G, lane = tid % G;
  uint32_t acc = 0;
  for (uint32_t it = 0; it < iters; ++it) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t row = hash32(grp * 0x9e3779b1U + it * U + u) % rows;
      v[u] = *reinterpret_cast<const u32x4*>(table + (size_t)row * R + lane * 16u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  sink[tid] = acc;
}

// 32 lanes per random 128-byte row: fp32 adds (one channel per lane) or packed-bf16 adds
// (two channels per lane, 64 per row).
template <bool BF16>
__global__ __launch_bounds__(kThreads) void atomic_probe(void* __restrict__ table, uint32_t rows,
                                                        uint32_t iters) {
  const uint32_t tid = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t grp = tid / 32u, lane = tid % 32u;
  for (uint32_t it = 0; it < iters; ++it) {
    const uint32_t row = hash32(grp * 0x9e3779b1U + it) % rows;
    if constexpr (BF16) {
      typedef short short2_t __attribute__((ext_vector_type(2)));
      typedef __attribute__((address_space(1))) short2_t* gptr;
      const gptr p = (gptr)(static_cast<char*>(table) + (size_t)row * 128u + lane * 4u);
      const short2_t one = {(short)0x3f80, (short)0x3f80};  // bf16 1.0, 1.0
      __builtin_amdgcn_global_atomic_fadd_v2bf16(p, one);
    } else {
      atomicAdd(reinterpret_cast<float*>(static_cast<char*>(table) + (size_t)row * 128u) + lane, 1.0f);
    }
  }
}

// LDS: MODE 0 ds_add_u32, 1 ds_add_f32, 2 plain stores, at random words of 16 K words.
template <int MODE>
__global__ __launch_bounds__(kThreads) void lds_probe(uint32_t iters, uint32_t* __restrict__ sink) {
  __shared__ uint32_t s[16384];
  for (int i = threadIdx.x; i < 16384; i += kThreads) s[i] = 0;
  __syncthreads();
  const uint32_t seed = blockIdx.x * kThreads + threadIdx.x;
  for (uint32_t it = 0; it < iters; ++it) {
    const uint32_t a = hash32(seed * 0x9e3779b1U + it) & 16383u;
    if constexpr (MODE == 0) atomicAdd(&s[a], 1u);
    else if constexpr (MODE == 1) atomicAdd(reinterpret_cast<float*>(&s[a]), 1.0f);
    else s[a] = it;
  }
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = s[seed & 16383u];
}

}  // namespace

extern "C" {

// kind: 64 or 128 (row bytes). Returns a HIP status.
int probe_gather(const void* table, uint64_t table_bytes, int row_bytes, uint32_t blocks,
                 uint32_t iters, uint32_t* sink, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t rows = (uint32_t)(table_bytes / (uint64_t)row_bytes);
  if (row_bytes == 64)
    hipLaunchKernelGGL((gather_probe<64, 8>), dim3(blocks), dim3(kThreads), 0, s,
                       static_cast<const char*>(table), rows, iters, sink);
  else if (row_bytes == 128)
    hipLaunchKernelGGL((gather_probe<128, 8>), dim3(blocks), dim3(kThreads), 0, s,
                       static_cast<const char*>(table), rows, iters, sink);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

int probe_atomic(void* table, uint64_t table_bytes, int bf16, uint32_t blocks, uint32_t iters,
                 void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t rows = (uint32_t)(table_bytes / 128u);
  if (bf16)
    hipLaunchKernelGGL(atomic_probe<true>, dim3(blocks), dim3(kThreads), 0, s, table, rows, iters);
  else
    hipLaunchKernelGGL(atomic_probe<false>, dim3(blocks), dim3(kThreads), 0, s, table, rows, iters);
  return (int)hipGetLastError();
}

int probe_lds(int mode, uint32_t blocks, uint32_t iters, uint32_t* sink, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mode == 0) hipLaunchKernelGGL(lds_probe<0>, dim3(blocks), dim3(kThreads), 0, s, iters, sink);
  else if (mode == 1) hipLaunchKernelGGL(lds_probe<1>, dim3(blocks), dim3(kThreads), 0, s, iters, sink);
  else hipLaunchKernelGGL(lds_probe<2>, dim3(blocks), dim3(kThreads), 0, s, iters, sink);
  return (int)hipGetLastError();
}

}  // extern "C"
