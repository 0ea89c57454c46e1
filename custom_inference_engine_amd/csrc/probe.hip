// Measurement helper: the HBM read ceiling for a paged access pattern.
//
// Reads n_chunks chunks of chunk_bytes each (chunk i at base + ids[i] *
// chunk_bytes), 16 bytes per lane per load, four chunks in flight per
// wavefront, and folds the data into one word so the loads cannot be
// removed.  With the chunk size of a KV page-head (2 KiB) and shuffled ids it
// is the paged decode's memory traffic without any of its math, i.e. the
// attainable bandwidth the decode kernel is judged against.
#include "cie_common.h"

namespace cie {

__global__ __launch_bounds__(256) void gather_read_kernel(const u32x4* __restrict__ base,
                                                          const int32_t* __restrict__ ids,
                                                          int64_t n_chunks, int per_chunk16,
                                                          uint32_t* sink) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) / kWave;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t c = wave * 4; c < n_chunks; c += n_waves * 4) {
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = u32x4{0u, 0u, 0u, 0u};
      if (c + j < n_chunks) {
        const u32x4* p = base + (int64_t)ids[c + j] * per_chunk16;
        for (int k = lane; k < per_chunk16; k += kWave) v[j] ^= p[k];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc ^= v[j];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[0] = 1u;
}

}  // namespace cie

using namespace cie;

extern "C" int cie_probe_gather_read(const void* base, const int32_t* chunk_ids, int64_t n_chunks,
                                     int64_t chunk_bytes, int64_t n_workgroups, uint32_t* sink,
                                     void* stream) {
  if (!base || !chunk_ids || !sink || n_chunks < 0 || chunk_bytes <= 0 || chunk_bytes % 1024 ||
      n_workgroups <= 0 || n_workgroups > 0x7fffffff)
    return CIE_EINVAL;
  if (reinterpret_cast<uintptr_t>(base) & 15) return CIE_EINVAL;
  if (n_chunks == 0) return CIE_OK;
  hipLaunchKernelGGL(gather_read_kernel, dim3((unsigned)n_workgroups), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(base), chunk_ids,
                     n_chunks, (int)(chunk_bytes / 16), sink);
  return (int)hipGetLastError();
}
