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
// Work.  A sequence's rows are cut into 16-row query tiles (the reference's
// BLOCK_M; grid (cdiv(max_seqlen, 16), H_kv, B), attn/core.py:90).  A tile's
// work is laid out as (row, head) columns, G heads per row, packed 16 to an
// MFMA column tile (attn_engine.h), so K/V bytes are shared by every head and
// row of the tile inside the MFMA.  The tile's key range [0, kv_len + last row
// + 1) is cut into up to kMaxChunks chunks, one workgroup each; the chunk's
// key tiles are split over the workgroup's waves, and every wave carries all
// of the tile's column tiles (in groups of kColGroup) for its keys, so each
// K/V byte is loaded once per workgroup and reused by every column in
// registers.  The waves fold their states through LDS one column tile at a
// time.  Chunks are short for decode-like tiles (<= 16 columns, memory-bound)
// and longer for prefill tiles (MFMA / VALU-bound), to bound partial traffic.
// A tile with one chunk writes o directly.  Otherwise each chunk writes its
// partial (m, l, acc) per column with device-coherent stores and the last
// chunk to arrive (counter per tile) merges them with log-sum-exp, writes o
// and resets the counter.  The reference instead walks a tile's whole prefix
// with one program and pads every L = 1 sequence to a 16-row tile
// (prefill_attention.py:49-50, 93).
#include "attn_engine.h"

namespace cie {

// Build-time tuning (defaults are the shipped configuration):
//   CIE_MIXED_CG           column tiles a wave carries at once (D = 64)
//   CIE_MIXED_SHORT_PAIRS  32-key steps per chunk of a short (<= 16 column) tile
//   CIE_MIXED_LONG_PAIRS   32-key steps per chunk of a prefill tile
//   CIE_MIXED_WG_PER_CU    workgroups per CU in the grid
#ifndef CIE_MIXED_CG
#define CIE_MIXED_CG 8
#endif
#ifndef CIE_MIXED_SHORT_PAIRS
#define CIE_MIXED_SHORT_PAIRS 16
#endif
#ifndef CIE_MIXED_LONG_PAIRS
#define CIE_MIXED_LONG_PAIRS 24
#endif
#ifndef CIE_MIXED_WG_PER_CU
#define CIE_MIXED_WG_PER_CU 2
#endif

constexpr int kMixedWaves = 4;
constexpr int kMaxChunks = 16;  // workgroups per query tile at most
constexpr int kShortPairsPerChunk = CIE_MIXED_SHORT_PAIRS;
constexpr int kLongPairsPerChunk = CIE_MIXED_LONG_PAIRS;
constexpr int kMaxCols = 128;  // columns per tile: 16 rows x G <= 8 heads

// Column tiles a wave carries at once (registers: 16*NT accumulators each).
template <int D>
constexpr int col_group() {
  return D <= 64 ? CIE_MIXED_CG : 2;
}

struct MixedParams {
  f16* o;
  const f16* q;
  const f16* k_pool;
  const f16* v_pool;
  const int64_t* cu_seqlens;
  const int64_t* kv_lens;
  const int64_t* slot_ids;
  const int64_t* block_table;
  float* part_m;  // [total_T][H_q][kMaxChunks]
  float* part_l;
  float* part_acc;  // [total_T][H_q][kMaxChunks][D]
  int32_t* counters;  // [B][H_kv][n_qtiles], zero between calls
  int64_t pool_page_stride, pool_head_stride, bt_stride, n_pages, total_T;
  int32_t bt_width, n_slots, B, H_q, H_kv, G, page_size, n_qtiles;
  float scale_log2;
  int32_t* err;
};

struct SeqInfo {
  int64_t t0;  // first packed row
  int64_t slot;
  int L;  // query rows
  int c;  // prior kv length
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
  int row0, rows, n_combos, n_ctiles, key_end, n_ktiles, n_chunks;
  bool shorttile;
};

__device__ __forceinline__ TilePlan tile_plan(int qt, const SeqInfo& s, int G) {
  TilePlan t;
  t.row0 = qt * 16;
  t.rows = min(16, s.L - t.row0);
  t.n_combos = t.rows * G;
  t.n_ctiles = (t.n_combos + 15) >> 4;
  t.key_end = s.c + t.row0 + t.rows;
  t.n_ktiles = (t.key_end + 15) >> 4;
  t.shorttile = t.n_ctiles == 1;
  const int n_pairs = (t.n_ktiles + 1) >> 1;
  const int per = t.shorttile ? kShortPairsPerChunk : kLongPairsPerChunk;
  t.n_chunks = max(1, min(kMaxChunks, (n_pairs + per - 1) / per));
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

// Global (row, q head) index of column cc of the tile.
__device__ __forceinline__ int64_t column_row(const MixedParams& p, const SeqInfo& s,
                                              const TilePlan& tp, int g, int cc) {
  const int row = cc / p.G;
  const int head = cc - row * p.G;
  return (s.t0 + tp.row0 + row) * p.H_q + g * p.G + head;
}

// Last chunk of a tile: combine the n_chunks partials of every column into o.
// A thread takes 16 consecutive dims of one column and issues all of its
// chunk loads at once; m / l of every (column, chunk) are staged in LDS
// (sm: >= 2 * kMaxCols * kMaxChunks floats).
template <int D>
__device__ __forceinline__ void merge_tile(const MixedParams& p, const SeqInfo& s,
                                           const TilePlan& tp, int g, float* sm) {
  const int K = tp.n_chunks;
  float* sm_m = sm;
  float* sm_l = sm + kMaxCols * kMaxChunks;
  for (int i = threadIdx.x; i < tp.n_combos * K; i += kMixedWaves * kWave) {
    const int cc = i / K;
    const int k = i - cc * K;
    const int64_t prow = column_row(p, s, tp, g, cc) * kMaxChunks + k;
    sm_m[i] = agent_load(p.part_m + prow);
    sm_l[i] = agent_load(p.part_l + prow);
  }
  __syncthreads();
  constexpr int kSeg = 16;  // dims per thread
  for (int it = threadIdx.x; it < tp.n_combos * (D / kSeg); it += kMixedWaves * kWave) {
    const int cc = it / (D / kSeg);
    const int d0 = (it - cc * (D / kSeg)) * kSeg;
    const int64_t crow = column_row(p, s, tp, g, cc);
    float M = kNegInf;
    for (int k = 0; k < K; ++k) M = fmaxf(M, sm_m[cc * K + k]);
    float num[kSeg] = {};
    float den = 0.f;
    // chunks in groups of 4: each group's loads are issued together
    for (int k0 = 0; k0 < K; k0 += 4) {
      float val[4][kSeg];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < kSeg; ++j)
          val[u][j] = k0 + u < K ? agent_load(p.part_acc + (crow * kMaxChunks + k0 + u) * D + d0 + j)
                                 : 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (k0 + u < K) {
          const float mk = sm_m[cc * K + k0 + u];
          const float a = mk == kNegInf ? 0.f : fast_exp2(mk - M);
          den += a * sm_l[cc * K + k0 + u];
#pragma unroll
          for (int j = 0; j < kSeg; ++j) num[j] += a * val[u][j];
        }
      }
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    f16x8 out[kSeg / 8];
#pragma unroll
    for (int j = 0; j < kSeg; ++j) out[j >> 3][j & 7] = (f16)(num[j] * inv);
#pragma unroll
    for (int v = 0; v < kSeg / 8; ++v) reinterpret_cast<f16x8*>(p.o + crow * D + d0)[v] = out[v];
  }
}

// One wave's share of a chunk: key tiles [w0, w1) against column tiles
// [ct0, ct0 + NCT); then the workgroup folds each column tile through LDS
// and writes o (single chunk) or the chunk's partial state.
template <int D, int NCT>
__device__ __forceinline__ void run_group(const MixedParams& p, const SeqInfo& s,
                                          const TilePlan& tp, int g, int ct0, int chunk, int w0,
                                          int w1, const PagedSrc& src, int wave, int r16, int grp,
                                          float (*sm_m)[16], float (*sm_l)[16],
                                          float (*sm_acc)[16][D + 1]) {
  constexpr int NT = Geo<D>::NT;
  f16x8 qop[NCT][Geo<D>::KS];
  int lim[NCT];
#pragma unroll
  for (int c = 0; c < NCT; ++c) load_combo_q<D>(p, s, tp, g, ct0 + c, r16, grp, qop[c], lim[c]);
  SoftmaxAcc<D, NCT> st;
  st.init();
  stream_tiles<D, NCT>(st, qop, lim, w0, w1, tp.key_end, src, p.scale_log2, r16, grp);
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const float l = col_sum4(st.l[c]);
    __syncthreads();  // the previous column tile's fold has read the LDS
    if (grp == 0) {
      sm_m[wave][r16] = st.m[c];
      sm_l[wave][r16] = l;
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) sm_acc[wave][r16][acc_dim<D>(grp, r, nt)] = st.acc[c][nt][r];
    __syncthreads();
    const int n_cols = min(16, tp.n_combos - (ct0 + c) * 16);
    for (int it = threadIdx.x; it < n_cols * D; it += kMixedWaves * kWave) {
      const int j = it / D;
      const int d = it - j * D;
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < kMixedWaves; ++w) M = fmaxf(M, sm_m[w][j]);
      float num = 0.f, den = 0.f;
#pragma unroll
      for (int w = 0; w < kMixedWaves; ++w) {
        const float mw = sm_m[w][j];
        if (mw != kNegInf) {
          const float a = fast_exp2(mw - M);
          num += a * sm_acc[w][j][d];
          den += a * sm_l[w][j];
        }
      }
      const int64_t crow = column_row(p, s, tp, g, (ct0 + c) * 16 + j);
      if (tp.n_chunks == 1) {
        p.o[crow * D + d] = (f16)(den > 0.f ? num / den : 0.f);
      } else {
        const int64_t prow = crow * kMaxChunks + chunk;
        agent_store(p.part_acc + prow * D + d, num);
        if (d == 0) {
          agent_store(p.part_m + prow, M);
          agent_store(p.part_l + prow, den);
        }
      }
    }
  }
}

constexpr int kMaxSeqs = 1024;  // sequences a launch can plan (LDS prefix table)

// Profiling builds only (-DCIE_MIXED_TRACE): thread 0 stamps each work item's
// phases (s_memrealtime) into the buffer passed as `err`, 8 words per
// (kv head, item).
#ifdef CIE_MIXED_TRACE
#define MIXED_TRACE(item, k, v)                                                                 \
  do {                                                                                          \
    if (threadIdx.x == 0 && p.err != nullptr && (item) < 4096) {                                \
      __builtin_amdgcn_s_waitcnt(0);                                                            \
      reinterpret_cast<uint64_t*>(p.err)[((int64_t)blockIdx.y * 4096 + (item)) * 8 + (k)] = (v); \
    }                                                                                           \
  } while (0)
#else
#define MIXED_TRACE(item, k, v) \
  do {                          \
  } while (0)
#endif

// Items of sequence s: sum over its (grid-covered) query tiles of the chunks.
__device__ __forceinline__ int seq_items(const SeqInfo& s, int n_qtiles, int G) {
  const int n_tiles = min((s.L + 15) >> 4, n_qtiles);
  int n = 0;
  for (int qt = 0; qt < n_tiles; ++qt) n += tile_plan(qt, s, G).n_chunks;
  return n;
}

// One work item: chunk `chunk` of query tile qt of sequence b, kv head g.
template <int D>
__device__ __forceinline__ void process_item(const MixedParams& p, const SeqInfo& s, int b, int g,
                                             int qt, int chunk, float (*sm_m)[16],
                                             float (*sm_l)[16], float (*sm_acc)[16][D + 1],
                                             int* sm_last, int item) {
  constexpr int CG = col_group<D>();
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r16 = lane & 15;
  const int grp = lane >> 4;
  const TilePlan tp = tile_plan(qt, s, p.G);
  // this chunk's key tiles, and this wave's share of them
  const int kt0 = (int)((int64_t)tp.n_ktiles * chunk / tp.n_chunks);
  const int kt1 = (int)((int64_t)tp.n_ktiles * (chunk + 1) / tp.n_chunks);
  const int w0 = kt0 + (int)((int64_t)(kt1 - kt0) * wave / kMixedWaves);
  const int w1 = kt0 + (int)((int64_t)(kt1 - kt0) * (wave + 1) / kMixedWaves);
  const PagedSrc src{p.k_pool,  p.v_pool,  p.block_table + s.slot * p.bt_stride,
                     (int64_t)g * p.pool_head_stride, p.pool_page_stride, p.n_pages,
                     p.page_size, p.err};

  for (int ct0 = 0; ct0 < tp.n_ctiles; ct0 += CG) {
    const int n = min(CG, tp.n_ctiles - ct0);
    switch (n) {
#define CIE_GROUP_CASE(k)                                                                      \
  case k:                                                                                      \
    if constexpr (k <= CG)                                                                     \
      run_group<D, k>(p, s, tp, g, ct0, chunk, w0, w1, src, wave, r16, grp, sm_m, sm_l, sm_acc); \
    break;
      CIE_GROUP_CASE(1)
      CIE_GROUP_CASE(2)
      CIE_GROUP_CASE(3)
      CIE_GROUP_CASE(4)
      CIE_GROUP_CASE(5)
      CIE_GROUP_CASE(6)
      CIE_GROUP_CASE(7)
      CIE_GROUP_CASE(8)
#undef CIE_GROUP_CASE
      default:
        break;
    }
  }
  MIXED_TRACE(item, 2, __builtin_amdgcn_s_memrealtime());
  MIXED_TRACE(item, 5, (uint64_t)(tp.n_ctiles * 1000000 + tp.n_chunks * 10000 + (kt1 - kt0)));
  if (tp.n_chunks == 1) {
    __syncthreads();  // LDS is reused by the next item
    MIXED_TRACE(item, 3, __builtin_amdgcn_s_memrealtime());
    return;
  }
  // The last chunk of this tile to arrive merges all chunks.
  int32_t* ctr = p.counters + ((int64_t)b * p.H_kv + g) * p.n_qtiles + qt;
  if (arrive_last(ctr, tp.n_chunks, sm_last)) {
    MIXED_TRACE(item, 4, __builtin_amdgcn_s_memrealtime());
    merge_tile<D>(p, s, tp, g, &sm_acc[0][0][0]);
    if (threadIdx.x == 0) *ctr = 0;
  }
  __syncthreads();
  MIXED_TRACE(item, 3, __builtin_amdgcn_s_memrealtime());
}

// Grid (n_workgroups, H_kv): every workgroup plans the whole batch — per
// sequence item counts and their prefix sums in LDS — and takes items
// blockIdx.x, blockIdx.x + gridDim.x, ...  (items ordered by sequence, tile,
// chunk), so no workgroup is launched for an empty (tile, chunk) slot.
template <int D>
__global__ __launch_bounds__(kMixedWaves * kWave) void mixed_attention_kernel(MixedParams p) {
  static_assert(kMixedWaves * 16 * (D + 1) >= 2 * kMaxCols * kMaxChunks, "merge scratch");
  __shared__ float sm_m[kMixedWaves][16];
  __shared__ float sm_l[kMixedWaves][16];
  __shared__ float sm_acc[kMixedWaves][16][D + 1];
  __shared__ int sm_last;
  __shared__ int sm_prefix[kMaxSeqs + 1];
  __shared__ int sm_scan[kMixedWaves * kWave];

  const int g = blockIdx.y;
  constexpr int NTH = kMixedWaves * kWave;
  // Per-thread item counts of sequences b = tid, tid + NTH, ... (B <= kMaxSeqs).
  int base = 0;
  for (int b0 = 0; b0 < p.B; b0 += NTH) {
    const int b = b0 + threadIdx.x;
    int n = 0;
    if (b < p.B) {
      const SeqInfo s = seq_info(p, b);
      if (g == 0 && blockIdx.x == 0 && ((s.L + 15) >> 4) > p.n_qtiles)
        set_err(p.err, CIE_ERRBIT_LEN);  // rows past max_seqlen are not computed
      n = s.L > 0 ? seq_items(s, p.n_qtiles, p.G) : 0;
    }
    // inclusive block scan of n
    sm_scan[threadIdx.x] = n;
    __syncthreads();
    for (int off = 1; off < NTH; off <<= 1) {
      const int add = threadIdx.x >= off ? sm_scan[threadIdx.x - off] : 0;
      __syncthreads();
      sm_scan[threadIdx.x] += add;
      __syncthreads();
    }
    if (b < p.B) sm_prefix[b + 1] = base + sm_scan[threadIdx.x];
    base += sm_scan[NTH - 1];
    __syncthreads();
  }
  if (threadIdx.x == 0) sm_prefix[0] = 0;
  __syncthreads();
  const int total = sm_prefix[p.B];
  MIXED_TRACE(blockIdx.x, 6, __builtin_amdgcn_s_memrealtime());  // planning done (first item slot)

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    MIXED_TRACE(item, 0, __builtin_amdgcn_s_memrealtime());
    // sequence: last b with prefix[b] <= item (binary search)
    int lo = 0, hi = p.B;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (sm_prefix[mid] <= item) lo = mid;
      else hi = mid;
    }
    const int b = lo;
    const SeqInfo s = seq_info(p, b);
    int j = item - sm_prefix[b];
    int qt = 0;
    for (;; ++qt) {
      const int nc = tile_plan(qt, s, p.G).n_chunks;
      if (j < nc) break;
      j -= nc;
    }
    MIXED_TRACE(item, 1, __builtin_amdgcn_s_memrealtime());
    MIXED_TRACE(item, 7, (uint64_t)(b * 1000 + qt));
    process_item<D>(p, s, b, g, qt, j, sm_m, sm_l, sm_acc, &sm_last, item);
  }
}

// Workgroups of the mixed grid: about two per CU over the kv heads.
static int mixed_workgroups(int H_kv) {
  int dev = 0, n_cu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  const int n = n_cu * CIE_MIXED_WG_PER_CU / H_kv;
  return n > 1 ? n : 1;
}

template <int D>
static int launch_mixed(const MixedParams& p, hipStream_t stream) {
  dim3 grid(mixed_workgroups(p.H_kv), p.H_kv, 1);
  hipLaunchKernelGGL((mixed_attention_kernel<D>), grid, dim3(kMixedWaves * kWave), 0, stream, p);
  return (int)hipGetLastError();
}

// partials: part_m | part_l | part_acc, each region 256-byte aligned
struct MixedLayout {
  int64_t m, l, acc, total;
};

static MixedLayout mixed_layout(int64_t total_T, int64_t H_q, int64_t D) {
  auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  const int64_t rows = total_T * H_q * kMaxChunks;
  MixedLayout w;
  w.m = 0;
  w.l = up(rows * 4);
  w.acc = up(w.l + rows * 4);
  w.total = up(w.acc + rows * D * 4);
  return w;
}

}  // namespace cie

using namespace cie;

extern "C" int64_t cie_mixed_partials_bytes(int64_t total_T, int64_t H_q, int64_t D) {
  if (total_T < 0 || H_q <= 0 || D <= 0) return -1;
  return mixed_layout(total_T, H_q, D).total;
}

extern "C" int64_t cie_mixed_counters(int64_t B, int64_t H_kv, int64_t max_seqlen) {
  if (B < 0 || H_kv <= 0 || max_seqlen < 0) return -1;
  return B * H_kv * ((max_seqlen + 15) / 16);
}

extern "C" int cie_mixed_attention(void* o, const void* q, const void* k_pool, const void* v_pool,
                                   const int64_t* cu_seqlens, const int64_t* kv_lens,
                                   const int64_t* slot_ids, const int64_t* block_table,
                                   void* partials, int32_t* counters, int64_t B, int64_t total_T,
                                   int64_t max_seqlen, int64_t H_q, int64_t H_kv, int64_t D,
                                   int64_t page_size, int64_t n_pages, int64_t pool_page_stride,
                                   int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
                                   int64_t n_slots, int32_t* err, void* stream) {
  if (B < 0 || total_T < 0 || max_seqlen < 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 ||
      n_pages <= 0 || bt_width <= 0 || bt_stride < bt_width || n_slots <= 0 || page_size <= 0)
    return CIE_EINVAL;
  if (B == 0 || total_T == 0 || max_seqlen == 0) return CIE_OK;
  if (!o || !q || !k_pool || !v_pool || !cu_seqlens || !kv_lens || !slot_ids || !block_table ||
      !partials || !counters)
    return CIE_EINVAL;
  const int64_t G = H_q / H_kv;
  const int64_t n_qtiles = (max_seqlen + 15) / 16;
  if (G > 8 || page_size % 16 != 0 || B > kMaxSeqs || H_kv > 65535 ||
      n_qtiles * kMaxChunks > 0x7fffffff || bt_width * page_size > 0x7fffffff ||
      total_T > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  if (D != 64 && D != 128) return CIE_EUNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(o) |
       reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool) |
       reinterpret_cast<uintptr_t>(partials) | reinterpret_cast<uintptr_t>(counters)) & 15)
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
  const MixedLayout w = mixed_layout(total_T, H_q, D);
  char* ws = static_cast<char*>(partials);
  p.part_m = reinterpret_cast<float*>(ws + w.m);
  p.part_l = reinterpret_cast<float*>(ws + w.l);
  p.part_acc = reinterpret_cast<float*>(ws + w.acc);
  p.counters = counters;
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_mixed<64>(p, st) : launch_mixed<128>(p, st);
}
