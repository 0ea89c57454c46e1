// Bench-only measurement helper (built into libcie_bench.so, never into the
// product library): the cost of the mixed kernel's 32-key step math with no
// memory traffic.
//
// cie_bench_step_probe runs `iters` steps of the math of one wave's 32-key
// step against 4 column tiles (D = 64) — the pipelined stream's segments:
// exponentials, P.V MFMAs and S MFMAs of the next step, then the reference-
// max check — on register-resident operands, with `waves_per_simd` waves
// per SIMD (one workgroup of 4 or 8 waves per CU, so the waves of a CU are
// co-resident; on all CUs or on n_cus of them), and returns the time per
// step (one wave's).
// Modes: 0 the whole step; 1 its 32 MFMAs alone; 2 its softmax VALU work
// alone (FMA, exponential, conversion, row sums).  Comparing 0 with 1 + 2
// shows how much of a lone wave's MFMA and VALU work overlaps; comparing
// waves_per_simd 1 and 2 what a second wave per SIMD adds.  No counterpart
// in the reference.
#include <vector>

#include "attn_engine.h"

namespace cie_bench {

using namespace cie;

template <int MODE, int THREADS>
__global__ __launch_bounds__(THREADS) void step_probe_kernel(float* out, int iters, float scale) {
  constexpr int D = 64, KS = 2, NT = 4, NCT = 4;
  const int lane = threadIdx.x & 63;
  SoftmaxAcc<D, NCT> st;
  st.init();
  f16x8 q[NCT][KS];
  KVPair<D> kv;
  for (int c = 0; c < NCT; ++c)
    for (int ks = 0; ks < KS; ++ks)
      for (int e = 0; e < 8; ++e) q[c][ks][e] = (f16)(0.01f * ((lane + c + ks + e) % 7));
  for (int t = 0; t < 2; ++t)
    for (int ks = 0; ks < KS; ++ks)
      for (int e = 0; e < 8; ++e) kv.k[t][ks][e] = (f16)(0.01f * ((lane * 3 + t + ks + e) % 5));
  for (int e = 0; e < 8; ++e)
    for (int d = 0; d < NT; ++d) kv.v[e][d] = (f16)(0.02f * ((lane + e + d) % 3));
  for (int c = 0; c < NCT; ++c) st.m[c] = 0.f;
  f32x4 s[NCT][2];
  for (int c = 0; c < NCT; ++c) {
    s[c][0] = f32x4{0.1f, 0.2f, 0.3f, 0.4f};
    s[c][1] = s[c][0];
  }
  for (int it = 0; it < iters; ++it) {
    asm volatile("" : "+v"(kv.k[0][0]), "+v"(kv.v[0]));  // a new step's operands
    if constexpr (MODE == 0) {
      f16x8 va[NT];
      v_operands<D>(va, kv);
      f32x4 s1[NCT][2];
      f16x8 pprev;
#pragma unroll
      for (int c = 0; c <= NCT; ++c) {
        __builtin_amdgcn_sched_barrier(0);
        f16x8 pc;
        if (c < NCT) pc = tile_probs(st.m[c], s[c], scale);
        if (c > 0) accumulate_probs<D, NCT>(st, c - 1, pprev, va);
        if (c < NCT) tile_scores_q<D>(s1[c], kv, q[c]);
        pprev = pc;
        if (CIE_STEP_INTERLEAVE && c > 0 && c < NCT) {
#pragma unroll
          for (int i = 0; i < NT + 2 * KS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      update_max<D, NCT>(st, s1, scale);
#pragma unroll
      for (int c = 0; c < NCT; ++c) {
        s[c][0] = s1[c][0];
        s[c][1] = s1[c][1];
      }
    } else if constexpr (MODE == 1) {
      f16x8 va[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) va[nt] = kv.k[0][nt & 1];
#pragma unroll
      for (int c = 0; c < NCT; ++c) {
        const f16x8 p = kv.k[1][c & 1];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) st.acc[c][nt] = mfma16x16x32(va[nt], p, st.acc[c][nt]);
        tile_scores_q<D>(s[c], kv, q[c]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < NCT; ++c) {
        const f16x8 pc = tile_probs(st.m[c], s[c], scale);
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        float l = st.lpart[c];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          l = __builtin_amdgcn_fdot2(h2{pc[2 * i], pc[2 * i + 1]}, h2{(f16)1.f, (f16)1.f}, l, false);
        st.lpart[c] = l;
        s[c][0] += 0.001f;
        s[c][1] -= 0.001f;
      }
    }
  }
  float acc = 0.f;
  for (int c = 0; c < NCT; ++c) {
    acc += st.l(c) + st.m[c] + s[c][0][0] + s[c][1][3];
    for (int nt = 0; nt < NT; ++nt) acc += st.acc[c][nt][0];
  }
  out[blockIdx.x * THREADS + threadIdx.x] = acc;  // keeps the work
}

}  // namespace cie_bench

using namespace cie_bench;

// 0 on success (*us_per_step set), -1 for bad arguments, else a hipError_t.
// Allocates and frees its own small output buffer; synchronizes the device.
// n_cus: CUs to occupy (0: all), so a run on a few CUs shows the step at the
// clock the chip keeps when few CUs draw power.
extern "C" int cie_bench_step_probe(int mode, int waves_per_simd, int iters, int n_cus,
                                    float* us_per_step) {
  if (mode < 0 || mode > 2 || waves_per_simd < 1 || waves_per_simd > 2 || iters < 1 || n_cus < 0 ||
      !us_per_step)
    return -1;
  int dev = 0, n_cu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  if (n_cus > 0 && n_cus < n_cu) n_cu = n_cus;
  // one workgroup per CU of 4 waves per wanted wave per SIMD, so the waves of
  // a CU are co-resident (the 512-thread kernel is built to fit two waves per
  // SIMD); n_cus workgroups land on n_cus different CUs
  const int blocks = n_cu;
  const int threads = 256 * waves_per_simd;
  float* out = nullptr;
  hipError_t e = hipMalloc(&out, (size_t)blocks * threads * sizeof(float));
  if (e != hipSuccess) return (int)e;
  hipEvent_t a = nullptr, b = nullptr;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  auto launch = [&](int n) {
    if (waves_per_simd == 1) {
      switch (mode) {
        case 0: hipLaunchKernelGGL((step_probe_kernel<0, 256>), dim3(blocks), dim3(256), 0, 0, out, n, 0.18f); break;
        case 1: hipLaunchKernelGGL((step_probe_kernel<1, 256>), dim3(blocks), dim3(256), 0, 0, out, n, 0.18f); break;
        default: hipLaunchKernelGGL((step_probe_kernel<2, 256>), dim3(blocks), dim3(256), 0, 0, out, n, 0.18f); break;
      }
    } else {
      switch (mode) {
        case 0: hipLaunchKernelGGL((step_probe_kernel<0, 512>), dim3(blocks), dim3(512), 0, 0, out, n, 0.18f); break;
        case 1: hipLaunchKernelGGL((step_probe_kernel<1, 512>), dim3(blocks), dim3(512), 0, 0, out, n, 0.18f); break;
        default: hipLaunchKernelGGL((step_probe_kernel<2, 512>), dim3(blocks), dim3(512), 0, 0, out, n, 0.18f); break;
      }
    }
  };
  launch(10);
  (void)hipEventRecord(a, 0);
  launch(iters);
  (void)hipEventRecord(b, 0);
  e = hipEventSynchronize(b);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
  if (e == hipSuccess) e = hipGetLastError();
  *us_per_step = ms * 1e3f / (float)iters;
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipFree(out);
  return (int)e;
}
