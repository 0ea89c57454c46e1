// Split-KV paged GQA decode for gfx950.
//
// Semantics follow decode_gqa_attention (attn/core.py:13-66): for sequence b,
// query head h (kv head g = h / G) attends the first lens[b] tokens of slot
// slot_ids[b]:  o = softmax(q . K^T * D^-0.5) . V, o = 0 when lens[b] == 0
// (the -inf guard of kernels/decode_attention.py:260-264).
//
// Work split.  Grid (n_splits, H_kv, B), WAVES wavefronts per workgroup.  The
// reference interleaves 16-row blocks over its P programs
// (kernels/decode_attention.py:71-75); here the ceil(L/16) key tiles of a
// (sequence, kv head) are cut into n_splits*WAVES contiguous, balanced runs, one
// per wave, so each wave streams a contiguous range of block-table entries.
// A wave keeps the G query heads of its kv head as MFMA columns (see
// attn_engine.h), the waves of a workgroup fold their softmax states through
// LDS, and the workgroup writes one partial (m, l, acc) per head for its
// split.  decode_merge_kernel then combines the splits with log-sum-exp,
// as kernels/decode_attention.py:243-264 does.
#include "attn_engine.h"

namespace cie {

struct DecodeParams {
  f16* o;
  const f16* q;
  const f16* k_pool;
  const f16* v_pool;
  const int64_t* lens;
  const int64_t* slot_ids;
  const int64_t* block_table;
  float* part_m;    // (B, H_q, S)
  float* part_l;    // (B, H_q, S)
  float* part_acc;  // (B, H_q, S, D)
  int64_t pool_page_stride, pool_head_stride, bt_stride, n_pages;
  int32_t bt_width, n_slots, B, H_q, H_kv, G, page_size, n_splits;
  float scale_log2;
  int32_t* err;
};

// Attended length of sequence b, clamped to what its block-table row can
// address; an invalid slot attends nothing.
__device__ __forceinline__ int decode_len(const DecodeParams& p, int b, int64_t& slot) {
  slot = p.slot_ids[b];
  if (slot < 0 || slot >= p.n_slots) {
    set_err(p.err, CIE_ERRBIT_PAGE);
    slot = 0;
    return 0;
  }
  int64_t L = p.lens[b];
  const int64_t cap = (int64_t)p.bt_width * p.page_size;
  if (L < 0 || L > cap) {
    set_err(p.err, CIE_ERRBIT_LEN);
    L = L < 0 ? 0 : cap;
  }
  return (int)L;
}

template <int D, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void decode_split_kernel(DecodeParams p) {
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];
  __shared__ float sm_acc[WAVES][16][D + 1];

  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r16 = lane & 15;
  const int grp = lane >> 4;

  int64_t slot;
  const int L = decode_len(p, b, slot);
  const int n_tiles = (L + 15) >> 4;
  const int total_waves = p.n_splits * WAVES;
  const int gw = split * WAVES + wave;
  const int t_begin = (int)((int64_t)n_tiles * gw / total_waves);
  const int t_end = (int)((int64_t)n_tiles * (gw + 1) / total_waves);

  // Q^T operand: column r16 = head g*G + r16 (zero past the group).
  f16x8 qop[1][KS];
  const f16* qrow = p.q + ((int64_t)b * p.H_q + g * p.G + r16) * D + 8 * grp;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qop[0][ks] = (r16 < p.G) ? *reinterpret_cast<const f16x8*>(qrow + 32 * ks) : f16x8{};
  const int lim[1] = {L};

  SoftmaxAcc<D, 1> st;
  st.init();

  const PagedSrc src{p.k_pool,  p.v_pool,  p.block_table + slot * p.bt_stride,
                     (int64_t)g * p.pool_head_stride, p.pool_page_stride, p.n_pages,
                     p.page_size, p.err};
  stream_tiles<D, 1>(st, qop, lim, t_begin, t_end, L, src, p.scale_log2, r16, grp);

  // Fold the waves of this workgroup.
  st.l[0] = col_sum4(st.l[0]);
  if (grp == 0) {
    sm_m[wave][r16] = st.m[0];
    sm_l[wave][r16] = st.l[0];
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm_acc[wave][r16][acc_dim<D>(grp, r, nt)] = st.acc[0][nt][r];
  __syncthreads();

  const int S = p.n_splits;
  for (int it = threadIdx.x; it < p.G * D; it += WAVES * kWave) {
    const int h = it / D;
    const int d = it - h * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][h]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float mw = sm_m[w][h];
      if (mw != kNegInf) {
        const float a = fast_exp2(mw - M);
        num += a * sm_acc[w][h][d];
        den += a * sm_l[w][h];
      }
    }
    const int64_t row = ((int64_t)b * p.H_q + g * p.G + h) * S + split;
    p.part_acc[row * D + d] = num;
    if (d == 0) {
      p.part_m[row] = M;
      p.part_l[row] = den;
    }
  }
}

// One wavefront per (query head, sequence): log-sum-exp merge of the splits.
template <int D>
__global__ __launch_bounds__(kWave) void decode_merge_kernel(DecodeParams p) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int S = p.n_splits;
  const int64_t row0 = ((int64_t)b * p.H_q + h) * S;
  float M = kNegInf;
  for (int s = 0; s < S; ++s) M = fmaxf(M, p.part_m[row0 + s]);
  for (int d = threadIdx.x; d < D; d += kWave) {
    float num = 0.f, den = 0.f;
    for (int s = 0; s < S; ++s) {
      const float ms = p.part_m[row0 + s];
      if (ms != kNegInf) {
        const float a = fast_exp2(ms - M);
        num += a * p.part_acc[(row0 + s) * D + d];
        den += a * p.part_l[row0 + s];
      }
    }
    const float out = (M == kNegInf) ? 0.f : num / den;
    p.o[((int64_t)b * p.H_q + h) * D + d] = (f16)out;
  }
}

constexpr int kDecodeWaves = 4;

template <int D>
static int launch_decode(const DecodeParams& p, hipStream_t stream) {
  dim3 grid(p.n_splits, p.H_kv, p.B);
  hipLaunchKernelGGL((decode_split_kernel<D, kDecodeWaves>), grid, dim3(kDecodeWaves * kWave),
                     0, stream, p);
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  hipLaunchKernelGGL((decode_merge_kernel<D>), dim3(p.H_q, p.B), dim3(kWave), 0, stream, p);
  return (int)hipGetLastError();
}

}  // namespace cie

using namespace cie;

extern "C" int64_t cie_paged_decode_workspace_bytes(int64_t B, int64_t H_q, int64_t D,
                                                    int64_t n_splits) {
  if (B < 0 || H_q <= 0 || D <= 0 || n_splits <= 0) return -1;
  return B * H_q * n_splits * (D + 2) * (int64_t)sizeof(float);
}

extern "C" int cie_paged_decode(void* o, const void* q, const void* k_pool, const void* v_pool,
                                const int64_t* lens, const int64_t* slot_ids,
                                const int64_t* block_table, void* workspace, int64_t B,
                                int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size,
                                int64_t n_pages, int64_t pool_page_stride,
                                int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
                                int64_t n_slots, int64_t n_splits, int32_t* err, void* stream) {
  if (B < 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || n_pages <= 0 || bt_width <= 0 ||
      bt_stride < bt_width || n_slots <= 0 || n_splits <= 0 || page_size <= 0)
    return CIE_EINVAL;
  if (B == 0) return CIE_OK;
  if (!o || !q || !k_pool || !v_pool || !lens || !slot_ids || !block_table || !workspace)
    return CIE_EINVAL;
  const int64_t G = H_q / H_kv;
  if (G > 16 || page_size % 16 != 0 || B > 65535 || H_kv > 65535 || n_splits > 65535 ||
      bt_width * page_size > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  if (D != 64 && D != 128) return CIE_EUNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_pool) |
       reinterpret_cast<uintptr_t>(v_pool)) & 15)
    return CIE_EINVAL;
  if (pool_page_stride % 8 != 0 || pool_head_stride % 8 != 0) return CIE_EINVAL;

  DecodeParams p{};
  p.o = static_cast<f16*>(o);
  p.q = static_cast<const f16*>(q);
  p.k_pool = static_cast<const f16*>(k_pool);
  p.v_pool = static_cast<const f16*>(v_pool);
  p.lens = lens;
  p.slot_ids = slot_ids;
  p.block_table = block_table;
  float* ws = static_cast<float*>(workspace);
  const int64_t rows = B * H_q * n_splits;
  p.part_m = ws;
  p.part_l = ws + rows;
  p.part_acc = ws + 2 * rows;
  p.pool_page_stride = pool_page_stride;
  p.pool_head_stride = pool_head_stride;
  p.bt_stride = bt_stride;
  p.n_pages = n_pages;
  p.bt_width = (int32_t)bt_width;
  p.n_slots = (int32_t)(n_slots > 0x7fffffff ? 0x7fffffff : n_slots);
  p.B = (int32_t)B;
  p.H_q = (int32_t)H_q;
  p.H_kv = (int32_t)H_kv;
  p.G = (int32_t)G;
  p.page_size = (int32_t)page_size;
  p.n_splits = (int32_t)n_splits;
  p.scale_log2 = kLog2e / __builtin_sqrtf((float)D);
  p.err = err;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_decode<64>(p, s) : launch_decode<128>(p, s);
}
