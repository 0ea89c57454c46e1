// Shared device helpers for the gfx950 paged-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cie_paged_attention.h"

namespace cie {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
// log2(e): softmax runs in the exp2 domain; scores are pre-multiplied by it.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float fast_exp2(float x) {
  // v_exp_f32: exact 2^x for x = -inf (gives 0), full-rate transcendental.
  return __builtin_amdgcn_exp2f(x);
}

// Lane exchange l <-> l^m (ds_bpermute under the hood).
__device__ __forceinline__ float lane_xor(float x, int m) {
  return __shfl_xor(x, m, kWave);
}

// max / sum over the four lanes {l, l^16, l^32, l^48}, i.e. over the lanes
// that hold the same MFMA output column (l % 16).
__device__ __forceinline__ float col_max4(float x) {
  x = fmaxf(x, lane_xor(x, 16));
  return fmaxf(x, lane_xor(x, 32));
}
__device__ __forceinline__ float col_sum4(float x) {
  x += lane_xor(x, 16);
  return x + lane_xor(x, 32);
}

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void set_err(int32_t* err, int bit) {
#ifndef CIE_DECODE_TRACE
  if (err) atomicOr(err, bit);
#endif
}

// Uniform (wave-invariant) value hint: lets the compiler keep it in an SGPR.
__device__ __forceinline__ int uniform(int x) {
  return __builtin_amdgcn_readfirstlane(x);
}
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

}  // namespace cie
