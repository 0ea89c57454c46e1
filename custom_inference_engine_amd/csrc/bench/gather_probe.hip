// Bench-only measurement helper (built into libcie_bench.so, never into the
// product library): the HBM read ceiling of a paged access pattern.
//
// cie_bench_gather_read reads n_chunks chunks of chunk_bytes each (chunk i at
// base + ids[i] * chunk_bytes), 16 bytes per lane per non-temporal load (the
// decode's V-row load policy, the fastest one measured for this pattern),
// four chunks in flight per wavefront, and folds the data into one word so
// the loads cannot be removed.  With the chunk size of a KV page-head
// (2 KiB) and shuffled ids it is the paged decode's memory traffic without
// any of its math: the attainable bandwidth the decode kernel is judged
// against.  No counterpart in the reference.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cie_bench {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kWave = 64;

template <int CHUNK16, int MAX_THREADS = 256>  // 16-byte words per chunk (a multiple of 64)
__global__ __launch_bounds__(MAX_THREADS) void gather_read_kernel(const u32x4* __restrict__ base,
                                                          const int32_t* __restrict__ ids,
                                                          int64_t n_chunks, uint32_t* sink) {
  constexpr int PER_LANE = CHUNK16 / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) / kWave;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t c = wave * 4; c < n_chunks; c += n_waves * 4) {
    u32x4 v[4][PER_LANE];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t id = (c + j < n_chunks) ? ids[c + j] : ids[c];
      const u32x4* p = base + id * CHUNK16;
#pragma unroll
      for (int k = 0; k < PER_LANE; ++k) v[j][k] = __builtin_nontemporal_load(p + k * kWave + lane);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int k = 0; k < PER_LANE; ++k) acc ^= v[j][k];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[0] = 1u;
}

}  // namespace cie_bench

using namespace cie_bench;

// 0 on success, -1 for bad arguments, -2 for an unsupported chunk size, else
// the hipError_t of the launch.
extern "C" int cie_bench_gather_read(const void* base, const int32_t* chunk_ids, int64_t n_chunks,
                                     int64_t chunk_bytes, int64_t n_workgroups, uint32_t* sink,
                                     void* stream) {
  if (!base || !chunk_ids || !sink || n_chunks < 0 || n_workgroups <= 0 ||
      n_workgroups > 0x7fffffff)
    return -1;
  if (reinterpret_cast<uintptr_t>(base) & 15) return -1;
  if (n_chunks == 0) return 0;
  const dim3 grid((unsigned)n_workgroups);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* b = static_cast<const u32x4*>(base);
  switch (chunk_bytes) {
    case 1024: hipLaunchKernelGGL(gather_read_kernel<64>, grid, dim3(256), 0, s, b, chunk_ids, n_chunks, sink); break;
    case 2048: hipLaunchKernelGGL(gather_read_kernel<128>, grid, dim3(256), 0, s, b, chunk_ids, n_chunks, sink); break;
    case 4096: hipLaunchKernelGGL(gather_read_kernel<256>, grid, dim3(256), 0, s, b, chunk_ids, n_chunks, sink); break;
    default: return -2;
  }
  return (int)hipGetLastError();
}

// The same read with `waves` wavefronts per workgroup (1..16), 2 KiB chunks:
// how many CUs the paged read needs (bench.py --probe-cus: the call's volume
// on 256 workgroups of 4 waves, 128 of 8, 64 of 16).  0 on success, -1 for
// bad arguments, else the hipError_t of the launch.
extern "C" int cie_bench_gather_read_waves(const void* base, const int32_t* chunk_ids,
                                           int64_t n_chunks, int64_t n_workgroups, int waves,
                                           uint32_t* sink, void* stream) {
  if (!base || !chunk_ids || !sink || n_chunks < 0 || n_workgroups <= 0 ||
      n_workgroups > 0x7fffffff || waves < 1 || waves > 16)
    return -1;
  if (reinterpret_cast<uintptr_t>(base) & 15) return -1;
  if (n_chunks == 0) return 0;
  hipLaunchKernelGGL((gather_read_kernel<128, 1024>), dim3((unsigned)n_workgroups), dim3(64 * waves), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(base), chunk_ids,
                     n_chunks, sink);
  return (int)hipGetLastError();
}
