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
// Key index of an absent tile: past every limit, so all its scores are masked.
constexpr int kNoKey = 0x3fffffff;

__device__ __forceinline__ float fast_exp2(float x) {
  // v_exp_f32 (a quarter-rate transcendental): 2^x, exactly 0 at x = -inf.
  return __builtin_amdgcn_exp2f(x);
}

// Inclusive prefix sum over the wave's 64 lanes, by DPP (no LDS): shifts
// by 1, 2, 4 and 8 lanes within each row of 16 (lanes shifted in from before
// the row read 0), then lane 15's row total added into rows 1 and 3 and
// lane 31's running total into rows 2 and 3.  Every lane must be active.
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
  return v;
}

// Lane exchange l <-> l^m (ds_bpermute under the hood).
__device__ __forceinline__ float lane_xor(float x, int m) {
  return __shfl_xor(x, m, kWave);
}

// The two values a lane sees after v_permlane16_swap / v_permlane32_swap of x
// with itself: {x[l], x[l ^ 16]} and {x[l], x[l ^ 32]} (in some order).  Both
// are VALU lane permutes on gfx950, no LDS round trip.
__device__ __forceinline__ void swap16(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap32(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// max / sum over the four lanes {l, l^16, l^32, l^48}, i.e. over the lanes
// that hold the same MFMA output column (l % 16).  Every lane of the four
// gets the same bits (the two operands of each step are the same pair).
__device__ __forceinline__ float col_max4(float x) {
  float a, b;
  swap16(x, a, b);
  swap32(fmaxf(a, b), a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float col_sum4(float x) {
  float a, b;
  swap16(x, a, b);
  swap32(a + b, a, b);
  return a + b;
}

// RoPE (transformers' apply_rotary_pos_emb: x*cos + rotate_half(x)*sin) of 8
// dims i (lo) and their partners i + D/2 (hi): lo' = lo*c_lo - hi*s_lo,
// hi' = hi*c_hi + lo*s_hi.  A product of two fp16 values is exact in fp32, so
// each output is the exact two-term sum rounded once to fp32, then to fp16.
__device__ __forceinline__ void rope8(f16x8& lo, f16x8& hi, f16x8 c_lo, f16x8 c_hi, f16x8 s_lo,
                                      f16x8 s_hi) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x0 = (float)lo[j];
    const float x1 = (float)hi[j];
    float y0 = __builtin_fmaf(x0, (float)c_lo[j], -(x1 * (float)s_lo[j]));
    float y1 = __builtin_fmaf(x1, (float)c_hi[j], x0 * (float)s_hi[j]);
    // Round to fp32 first: without this barrier the compiler may fuse the
    // FMA and the fp16 conversion into one v_fma_mixlo_f16, which rounds the
    // exact sum straight to fp16 and differs from the reference's fp32 ->
    // fp16 double rounding in the last bit now and then.
    asm volatile("" : "+v"(y0), "+v"(y1));
    lo[j] = (f16)y0;
    hi[j] = (f16)y1;
  }
}

// A load of whole cache lines the kernel reads exactly once (V rows streamed
// by the decode): the non-temporal policy (global_load ... nt) keeps them
// from being allocated for reuse in the caches, which raises the HBM read
// rate of shuffled 2 KiB pages from ~5.8 to ~6.5 TB/s on MI355X.  Not for
// partial lines whose other part a later load reads: an operand-layout K
// load covers half of each 128-byte row and the next k-step the other half,
// and with nt that second half is fetched from HBM again (+4.5 % traffic and
// +0.5 us per decode call when K was loaded this way).
template <class T>
__device__ __forceinline__ T stream_load(const T* p) {
  return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void set_err(int32_t* err, int bit) {
  if (err) atomicOr(err, bit);
}

// Device-coherent (agent-scope) accesses: global_store / global_load with sc1,
// visible across workgroups on every XCD once the store has completed
// (s_waitcnt vmcnt(0)), with no L2 writeback / invalidate.
__device__ __forceinline__ void agent_store(float* ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float agent_load(const float* ptr) {
  return __hip_atomic_load(const_cast<float*>(ptr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte device-coherent accesses: buffer_load / buffer_store_dwordx4 with
// sc1 (the same cache policy as the agent-scope accesses above) through a
// raw buffer resource over [base, base + bytes).  base must be wave-uniform.
constexpr int kBufSc1 = 16;                  // cache-policy operand: sc1
constexpr int kBufRsrcWord3 = 0x00020000;    // raw 32-bit buffer (gfx9 family)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  // readfirstlane yields an int: widen through uint32_t, never sign-extend
  // the low word into the high one.
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const uint64_t u = ((uint64_t)hi << 32) | lo;
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), 0, (int)bytes, kBufRsrcWord3);
}
__device__ __forceinline__ void agent_store4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, kBufSc1);
}
__device__ __forceinline__ f32x4 agent_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kBufSc1));
}
// s_waitcnt vmcnt(0): every vector-memory access this wave issued has
// completed (stores included: on gfx9 they count in vmcnt).  The intrinsic
// touches no memory as far as LLVM is concerned, so compiler-only fences on
// both sides pin the agent-scope stores before it and the arrival atomic
// after it; tests/test_asm_order.py checks the order in the built code.
__device__ __forceinline__ void wait_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Split arrival counters.  A group of n_members workgroups that each store a
// partial result (with agent_store / agent_store4) elects its last arriver
// with one relaxed agent-scope fetch_add on the group's arrival word; the
// winner merges and puts the word back to zero, so a buffer of zeros stays
// zeros across stream-ordered calls.  Ordering (gfx950, LLVM AMDGPU memory
// model, GFX942 family): relaxed agent-scope stores, loads and RMWs are
// global_store / global_load / global_atomic with sc1, each coherent at agent
// scope by itself; the partial stores have completed (vmcnt(0)) before the
// atomic is issued, and the winner's sc1 loads are issued after the atomic
// returned, so they read the completed stores.  No L2 writeback
// (buffer_wbl2) or invalidate is needed, because no partial is ever accessed
// without sc1.
//
// A word outside [0, n_members) at the start of a call (a caller's unzeroed
// buffer, a call that overlapped another on the same counters) is detected:
// an arrival that reads such a value raises CIE_ERRBIT_SPLIT and counts
// itself on the group's stale word, n_words further on.  When every arrival
// of a call reads a stale value (the word held n_members or more, or was
// negative enough), the last of them puts both words back to zero, so the
// next call is clean; a stale value below n_members is not distinguishable
// from live arrivals and is reported only by the arrivals that overshoot.
__device__ __forceinline__ void counter_reset(int32_t* word) {
  __hip_atomic_store(word, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool arrive_last(int32_t* arrival, int64_t n_words, int n_members,
                                            int* sm_flag, int32_t* err) {
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(arrival, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *sm_flag = old == n_members - 1;
    if (old < 0 || old >= n_members) {
      if (err) atomicOr(err, CIE_ERRBIT_SPLIT);
      int32_t* stale = arrival + n_words;
      if (__hip_atomic_fetch_add(stale, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
          n_members - 1) {
        counter_reset(arrival);
        counter_reset(stale);
      }
    }
  }
  __syncthreads();
  return *sm_flag != 0;
}


// floor(x / d) for x * d < 2^31 as one multiply-high: magic = ceil(2^31 / d)
// (div_magic, computed on the host, so the kernel holds no per-lane
// reciprocal registers for a run-time divisor): 2x * magic / 2^32 =
// x / d + x * r / (d * 2^31) with r < d, whose floor is x / d exactly.
__device__ __forceinline__ int magic_div(int x, uint32_t magic) {
  return (int)__umulhi((uint32_t)x << 1, magic);
}
static inline uint32_t div_magic(uint32_t d) {
  return (uint32_t)((((uint64_t)1 << 31) + d - 1) / d);
}

// A value the compiler must treat as unknown at this point: what is derived
// from it is computed here, not hoisted to the kernel's start and held in
// registers across the hot loops.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Uniform (wave-invariant) value hint: lets the compiler keep it in an SGPR.
__device__ __forceinline__ int uniform(int x) {
  return __builtin_amdgcn_readfirstlane(x);
}
// 64-bit value held by lane l (l wave-uniform).
__device__ __forceinline__ int64_t readlane64(int64_t x, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)x, l);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)x >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

}  // namespace cie
