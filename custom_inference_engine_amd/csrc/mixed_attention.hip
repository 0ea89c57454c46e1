// Varlen causal GQA attention over the paged pool (chunked prefill + decode in
// one launch) for gfx950.
//
// Semantics follow mixed_gqa_attention (attn/core.py:69-111) and
// kernels/prefill_attention.py:37-198: sequence b owns query rows
// [cu_seqlens[b], cu_seqlens[b+1]); its row i sits at absolute position
// kv_lens[b] + i and attends keys 0 .. kv_lens[b] + i of slot slot_ids[b]
// (the causal rule kv_len + row >= key of prefill_attention.py:145-146).
// Rows outside every sequence are left untouched.
//
// A sequence's rows are cut into 16-row query tiles (the reference's BLOCK_M,
// grid (cdiv(max_seqlen, 16), H_kv, B), attn/core.py:90).  Each tile's work is
// laid out as (row, head) columns, G heads per row, packed 16 to an MFMA
// column tile (attn_engine.h), so K/V bytes are shared by every head and row
// of the tile inside the MFMA:
//  * prefill tiles (more than 16 columns): "row-parallel" — the workgroup's
//    waves take different column tiles and each streams the tile's whole key
//    range [0, kv_len + last row]; the result is written directly.
//  * short tiles (<= 16 columns: L = 1 decode rows, or a 1-2 row tail):
//    "key-parallel" — the key range is cut over up to kMixedSplits workgroups
//    and their waves, like the decode kernel.  Waves fold through LDS; with
//    more than one workgroup the partial states go to the workspace and
//    mixed_merge_kernel combines them.
// The reference instead pads every L = 1 sequence to a 16-row tile and walks
// its whole prefix with one program (prefill_attention.py:49-50, 93).
#include "attn_engine.h"

namespace cie {

constexpr int kMixedWaves = 4;
constexpr int kMixedSplits = 16;       // max workgroups per key-parallel tile
constexpr int kMinPairsPerSplit = 8;   // 32-key steps per key-parallel workgroup

struct MixedParams {
  f16* o;
  const f16* q;
  const f16* k_pool;
  const f16* v_pool;
  const int64_t* cu_seqlens;
  const int64_t* kv_lens;
  const int64_t* slot_ids;
  const int64_t* block_table;
  float* part_m;    // [B][H_kv][16 columns][kMixedSplits]
  float* part_l;
  float* part_acc;  // ... x D
  int64_t pool_page_stride, pool_head_stride, bt_stride, n_pages, total_T;
  int32_t bt_width, n_slots, B, H_q, H_kv, G, page_size, n_qtiles;
  float scale_log2;
  int32_t* err;
};

struct SeqInfo {
  int64_t t0;    // first packed row
  int64_t slot;
  int L;         // query rows
  int c;         // prior kv length
};

__device__ __forceinline__ SeqInfo seq_info(const MixedParams& p, int b) {
  SeqInfo s{0, 0, 0, 0};
  const int64_t t0 = p.cu_seqlens[b];
  const int64_t t1 = p.cu_seqlens[b + 1];
  const int64_t slot = p.slot_ids[b];
  const int64_t c = p.kv_lens[b];
  if (t0 < 0 || t1 < t0 || t1 > p.total_T || slot < 0 || slot >= p.n_slots) {
    if (t1 != t0) set_err(p.err, CIE_ERRBIT_PAGE);
    return s;
  }
  const int64_t cap = (int64_t)p.bt_width * p.page_size;
  if (c < 0 || c + (t1 - t0) > cap) {
    set_err(p.err, CIE_ERRBIT_LEN);
    return s;
  }
  s.t0 = t0;
  s.slot = slot;
  s.L = (int)(t1 - t0);
  s.c = (int)c;
  return s;
}

struct TilePlan {
  int row0, rows, n_combos, n_ctiles, key_end, n_ktiles, n_act;
  bool keypar;
};

__device__ __forceinline__ TilePlan tile_plan(int qt, const SeqInfo& s, int G) {
  TilePlan t;
  t.row0 = qt * 16;
  t.rows = min(16, s.L - t.row0);
  t.n_combos = t.rows * G;
  t.n_ctiles = (t.n_combos + 15) >> 4;
  t.key_end = s.c + t.row0 + t.rows;
  t.n_ktiles = (t.key_end + 15) >> 4;
  // Only a sequence's last tile may run key-parallel: the extra split
  // workgroups and the merge address partials by (sequence, column), one
  // short tile per sequence.  Full 16-row tiles with <= 16 columns (G = 1)
  // run row-parallel on one wave.
  t.keypar = t.n_ctiles == 1 && t.row0 + t.rows == s.L;
  const int n_pairs = (t.n_ktiles + 1) >> 1;
  t.n_act = t.keypar ? max(1, min(kMixedSplits, (n_pairs + kMinPairsPerSplit - 1) / kMinPairsPerSplit))
                     : 1;
  return t;
}

// Q^T operand and key limit of column tile ct (columns = (row, head) pairs).
template <int D>
__device__ __forceinline__ void load_combo_q(const MixedParams& p, const SeqInfo& s,
                                             const TilePlan& tp, int g, int ct, int r16, int grp,
                                             f16x8 (&qop)[Geo<D>::KS], int& lim) {
  const int cc = ct * 16 + r16;
  if (cc < tp.n_combos) {
    const int row = cc / p.G;
    const int head = cc - row * p.G;
    const f16* qrow =
        p.q + ((s.t0 + tp.row0 + row) * p.H_q + g * p.G + head) * (int64_t)D + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < Geo<D>::KS; ++ks) qop[ks] = *reinterpret_cast<const f16x8*>(qrow + 32 * ks);
    lim = s.c + tp.row0 + row + 1;
  } else {
#pragma unroll
    for (int ks = 0; ks < Geo<D>::KS; ++ks) qop[ks] = f16x8{};
    lim = tp.key_end;
  }
}

// Store a normalised output column (lane holds 4*NT consecutive dims).
template <int D>
__device__ __forceinline__ void store_column(const MixedParams& p, const SeqInfo& s,
                                             const TilePlan& tp, int g, int cc, int grp,
                                             const f32x4 (&acc)[Geo<D>::NT], float l) {
  constexpr int NT = Geo<D>::NT;
  if (cc >= tp.n_combos) return;
  const int row = cc / p.G;
  const int head = cc - row * p.G;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  f16* orow = p.o + ((s.t0 + tp.row0 + row) * p.H_q + g * p.G + head) * (int64_t)D + NT * 4 * grp;
  f16x8 out[NT / 2];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int i = NT * r + nt;
      out[i >> 3][i & 7] = (f16)(acc[nt][r] * inv);
    }
#pragma unroll
  for (int v = 0; v < NT / 2; ++v) reinterpret_cast<f16x8*>(orow)[v] = out[v];
}

template <int D, int NCT>
__device__ __forceinline__ void rowpar_wave(const MixedParams& p, const SeqInfo& s,
                                            const TilePlan& tp, int g, int ct_first,
                                            const PagedSrc& src, int r16, int grp) {
  f16x8 qop[NCT][Geo<D>::KS];
  int lim[NCT];
#pragma unroll
  for (int c = 0; c < NCT; ++c)
    load_combo_q<D>(p, s, tp, g, ct_first + c * kMixedWaves, r16, grp, qop[c], lim[c]);
  SoftmaxAcc<D, NCT> st;
  st.init();
  stream_tiles<D, NCT>(st, qop, lim, 0, tp.n_ktiles, tp.key_end, src, p.scale_log2, r16, grp);
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const float l = col_sum4(st.l[c]);
    store_column<D>(p, s, tp, g, (ct_first + c * kMixedWaves) * 16 + r16, grp, st.acc[c], l);
  }
}

template <int D>
__global__ __launch_bounds__(kMixedWaves * kWave) void mixed_attention_kernel(MixedParams p) {
  constexpr int NT = Geo<D>::NT;
  __shared__ float sm_m[kMixedWaves][16];
  __shared__ float sm_l[kMixedWaves][16];
  __shared__ float sm_acc[kMixedWaves][16][D + 1];

  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r16 = lane & 15;
  const int grp = lane >> 4;

  const SeqInfo s = seq_info(p, b);
  if (s.L == 0) return;
  // Rows past the grid's max_seqlen bound are not computed (as in the
  // reference's cdiv(max_seqlen, BLOCK_M) grid); report them.
  if (blockIdx.x == 0 && g == 0 && threadIdx.x == 0 && ((s.L + 15) >> 4) > p.n_qtiles)
    set_err(p.err, CIE_ERRBIT_LEN);
  // blockIdx.x < n_qtiles: split 0 of query tile blockIdx.x;
  // otherwise: extra split of the sequence's last tile (key-parallel only).
  int qt, split;
  if ((int)blockIdx.x < p.n_qtiles) {
    qt = blockIdx.x;
    split = 0;
  } else {
    qt = (s.L - 1) >> 4;
    split = blockIdx.x - p.n_qtiles + 1;
  }
  if (qt * 16 >= s.L || qt >= p.n_qtiles) return;
  const TilePlan tp = tile_plan(qt, s, p.G);
  if (split >= tp.n_act) return;

  const PagedSrc src{p.k_pool,  p.v_pool,  p.block_table + s.slot * p.bt_stride,
                     (int64_t)g * p.pool_head_stride, p.pool_page_stride, p.n_pages,
                     p.page_size, p.err};

  if (!tp.keypar) {
    // Row-parallel prefill tile: wave w owns column tiles w and w + kMixedWaves.
    if (wave >= tp.n_ctiles) return;
    if (wave + kMixedWaves < tp.n_ctiles)
      rowpar_wave<D, 2>(p, s, tp, g, wave, src, r16, grp);
    else
      rowpar_wave<D, 1>(p, s, tp, g, wave, src, r16, grp);
    return;
  }

  // Key-parallel short tile: this workgroup's waves split its key range.
  f16x8 qop[1][Geo<D>::KS];
  int lim[1];
  load_combo_q<D>(p, s, tp, g, 0, r16, grp, qop[0], lim[0]);
  SoftmaxAcc<D, 1> st;
  st.init();
  const int total_waves = tp.n_act * kMixedWaves;
  const int gw = split * kMixedWaves + wave;
  const int t_begin = (int)((int64_t)tp.n_ktiles * gw / total_waves);
  const int t_end = (int)((int64_t)tp.n_ktiles * (gw + 1) / total_waves);
  stream_tiles<D, 1>(st, qop, lim, t_begin, t_end, tp.key_end, src, p.scale_log2, r16, grp);

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

  for (int it = threadIdx.x; it < tp.n_combos * D; it += kMixedWaves * kWave) {
    const int cc = it / D;
    const int d = it - cc * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kMixedWaves; ++w) M = fmaxf(M, sm_m[w][cc]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kMixedWaves; ++w) {
      const float mw = sm_m[w][cc];
      if (mw != kNegInf) {
        const float a = fast_exp2(mw - M);
        num += a * sm_acc[w][cc][d];
        den += a * sm_l[w][cc];
      }
    }
    if (tp.n_act == 1) {
      const int row = cc / p.G;
      const int head = cc - row * p.G;
      p.o[((s.t0 + tp.row0 + row) * p.H_q + g * p.G + head) * (int64_t)D + d] =
          (f16)(den > 0.f ? num / den : 0.f);
    } else {
      const int64_t prow = (((int64_t)b * p.H_kv + g) * 16 + cc) * kMixedSplits + split;
      p.part_acc[prow * D + d] = num;
      if (d == 0) {
        p.part_m[prow] = M;
        p.part_l[prow] = den;
      }
    }
  }
}

// One wavefront per (sequence, kv head): merges the split partials of the
// sequence's last tile when it ran key-parallel over several workgroups.
template <int D>
__global__ __launch_bounds__(kWave) void mixed_merge_kernel(MixedParams p) {
  const int b = blockIdx.x;
  const int g = blockIdx.y;
  const SeqInfo s = seq_info(p, b);
  if (s.L == 0) return;
  const int qt = (s.L - 1) >> 4;
  if (qt >= p.n_qtiles) return;
  const TilePlan tp = tile_plan(qt, s, p.G);
  if (!tp.keypar || tp.n_act <= 1) return;
  for (int cc = 0; cc < tp.n_combos; ++cc) {
    const int64_t prow0 = (((int64_t)b * p.H_kv + g) * 16 + cc) * kMixedSplits;
    float M = kNegInf;
    for (int sp = 0; sp < tp.n_act; ++sp) M = fmaxf(M, p.part_m[prow0 + sp]);
    const int row = cc / p.G;
    const int head = cc - row * p.G;
    f16* orow = p.o + ((s.t0 + tp.row0 + row) * p.H_q + g * p.G + head) * (int64_t)D;
    for (int d = threadIdx.x; d < D; d += kWave) {
      float num = 0.f, den = 0.f;
      for (int sp = 0; sp < tp.n_act; ++sp) {
        const float ms = p.part_m[prow0 + sp];
        if (ms != kNegInf) {
          const float a = fast_exp2(ms - M);
          num += a * p.part_acc[(prow0 + sp) * D + d];
          den += a * p.part_l[prow0 + sp];
        }
      }
      orow[d] = (f16)(den > 0.f ? num / den : 0.f);
    }
  }
}

template <int D>
static int launch_mixed(const MixedParams& p, hipStream_t stream) {
  dim3 grid(p.n_qtiles + kMixedSplits - 1, p.H_kv, p.B);
  hipLaunchKernelGGL((mixed_attention_kernel<D>), grid, dim3(kMixedWaves * kWave), 0, stream, p);
  int rc = (int)hipGetLastError();
  if (rc) return rc;
  hipLaunchKernelGGL((mixed_merge_kernel<D>), dim3(p.B, p.H_kv), dim3(kWave), 0, stream, p);
  return (int)hipGetLastError();
}

}  // namespace cie

using namespace cie;

extern "C" int64_t cie_mixed_workspace_bytes(int64_t B, int64_t H_kv, int64_t D) {
  if (B < 0 || H_kv <= 0 || D <= 0) return -1;
  return B * H_kv * 16 * kMixedSplits * (D + 2) * (int64_t)sizeof(float);
}

extern "C" int cie_mixed_attention(void* o, const void* q, const void* k_pool, const void* v_pool,
                                   const int64_t* cu_seqlens, const int64_t* kv_lens,
                                   const int64_t* slot_ids, const int64_t* block_table,
                                   void* workspace, int64_t B, int64_t total_T,
                                   int64_t max_seqlen, int64_t H_q, int64_t H_kv, int64_t D,
                                   int64_t page_size, int64_t n_pages, int64_t pool_page_stride,
                                   int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
                                   int64_t n_slots, int32_t* err, void* stream) {
  if (B < 0 || total_T < 0 || max_seqlen < 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 ||
      n_pages <= 0 || bt_width <= 0 || bt_stride < bt_width || n_slots <= 0 || page_size <= 0)
    return CIE_EINVAL;
  if (B == 0 || total_T == 0 || max_seqlen == 0) return CIE_OK;
  if (!o || !q || !k_pool || !v_pool || !cu_seqlens || !kv_lens || !slot_ids || !block_table ||
      !workspace)
    return CIE_EINVAL;
  const int64_t G = H_q / H_kv;
  const int64_t n_qtiles = (max_seqlen + 15) / 16;
  if (G > 8 || page_size % 16 != 0 || B > 65535 || H_kv > 65535 ||
      n_qtiles + kMixedSplits > 0x7fffffff || bt_width * page_size > 0x7fffffff ||
      total_T > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  if (D != 64 && D != 128) return CIE_EUNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(o) |
       reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool)) & 15)
    return CIE_EINVAL;
  if (pool_page_stride % 8 != 0 || pool_head_stride % 8 != 0) return CIE_EINVAL;

  MixedParams p{};
  p.o = static_cast<f16*>(o);
  p.q = static_cast<const f16*>(q);
  p.k_pool = static_cast<const f16*>(k_pool);
  p.v_pool = static_cast<const f16*>(v_pool);
  p.cu_seqlens = cu_seqlens;
  p.kv_lens = kv_lens;
  p.slot_ids = slot_ids;
  p.block_table = block_table;
  float* ws = static_cast<float*>(workspace);
  const int64_t rows = B * H_kv * 16 * kMixedSplits;
  p.part_m = ws;
  p.part_l = ws + rows;
  p.part_acc = ws + 2 * rows;
  p.pool_page_stride = pool_page_stride;
  p.pool_head_stride = pool_head_stride;
  p.bt_stride = bt_stride;
  p.n_pages = n_pages;
  p.total_T = total_T;
  p.bt_width = (int32_t)bt_width;
  p.n_slots = (int32_t)(n_slots > 0x7fffffff ? 0x7fffffff : n_slots);
  p.B = (int32_t)B;
  p.H_q = (int32_t)H_q;
  p.H_kv = (int32_t)H_kv;
  p.G = (int32_t)G;
  p.page_size = (int32_t)page_size;
  p.n_qtiles = (int32_t)n_qtiles;
  p.scale_log2 = kLog2e / __builtin_sqrtf((float)D);
  p.err = err;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_mixed<64>(p, s) : launch_mixed<128>(p, s);
}
