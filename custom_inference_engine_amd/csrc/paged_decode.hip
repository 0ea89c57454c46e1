// Split-KV paged GQA decode for gfx950: one launch per call.
//
// Semantics follow decode_gqa_attention (attn/core.py:13-66): for sequence b,
// query head h (kv head g = h / G) attends the first L tokens of slot
// slot_ids[b]: o = softmax(q . K^T * D^-0.5) . V, o = 0 when L == 0 (the
// -inf guard of kernels/decode_attention.py:260-264).
//
// Three entry modes share the kernel:
//  * plain  (cie_paged_decode): L = lens[b], the pool is read-only — the
//    reference's gqa_decode_attention op.
//  * append (cie_paged_decode_append): pos = lens_pool[slot], L = pos + 1; the
//    new token's K/V rows are written to (block_table[slot, pos / P], pos % P)
//    exactly as KVStorage.decode_update (kv_cache/storage.py:87-122) does, and
//    the wave that owns that tile reads them from k_new / v_new instead of the
//    pool, so the append costs no extra launch and no extra round trip.
//  * append + rope (cie_paged_decode_qkv_rope): q, k_new and v_new are column
//    blocks of the fused QKV projection's output row, and q and k_new are
//    rotated in registers (RoPE of transformers' apply_rotary_pos_emb, as
//    TritonQwen2Attention.forward applies it, attn/core.py:193-198) before use;
//    the pool receives the rotated K row.
//
// Work split.  Grid (n_splits, H_kv, B), WAVES wavefronts per workgroup.  The
// ceil(L/16) key tiles of a (sequence, kv head) are dealt round-robin over its
// TW = n_splits * WAVES waves: wave gw takes tiles gw, gw + TW, gw + 2*TW, ...
// (the reference also interleaves 16-row blocks over its P programs,
// kernels/decode_attention.py:71-75).  A wave keeps the G query heads of its
// kv head as MFMA columns (attn_engine.h); the waves of a workgroup fold their
// softmax states through LDS.  With one split the workgroup writes o
// directly.  Otherwise it writes a partial (m, l, acc) per head, and the last
// workgroup of the (sequence, kv head) to finish — elected on a device-scope
// arrival counter (arrive_last) — merges the splits with log-sum-exp as
// kernels/decode_attention.py:243-264 does, writes o and resets the counter
// to zero for the next call.
#include <mutex>

#include "attn_engine.h"

// Build-time tuning (defaults are the shipped configuration):
//   CIE_DECODE_WAVES  wavefronts per workgroup
//   CIE_DECODE_PF     32-key steps whose loads are in flight ahead of the math
#ifndef CIE_DECODE_WAVES
#define CIE_DECODE_WAVES 4
#endif
#ifndef CIE_DECODE_PF
#define CIE_DECODE_PF 1
#endif

namespace cie {

struct DecodeParams {
  f16* o;
  const f16* q;
  int64_t q_row_stride;  // elements between sequences' q rows (H_q * D when dense)
  const f16* cos;        // rope mode: (B, D) rows of the new token's cos / sin
  const f16* sin;
  int64_t cs_stride;
  f16* k_pool;
  f16* v_pool;
  const f16* k_new;  // append mode: (B, H_kv, D) rows with the strides below
  const f16* v_new;
  int64_t k_tok_stride, k_head_stride, v_tok_stride, v_head_stride;
  const int64_t* lens;  // plain: (B,) attended; append: (n_slots,) prior per slot
  const int64_t* slot_ids;
  const int64_t* block_table;
  float* part_m;    // (B, H_q, S)
  float* part_l;    // (B, H_q, S)
  float* part_acc;  // (B, H_q, S, D)
  int32_t* counters;  // 2 * (B * H_kv): arrival words, then stale words; zero between calls
  const int32_t* plan;  // planned launches: the step's plan (cie_paged_decode_plan)
  int32_t n_wg;         // planned launches: the grid (workgroups) the plan was made for
  int64_t pool_page_stride, pool_head_stride, bt_stride, n_pages;
  int32_t bt_width, n_slots, B, H_q, H_kv, G, page_size, n_splits;
  float scale_log2;
  int32_t* err;
};

// Append mode: point the lanes that hold key `pos` at the new rows instead of
// the pool, and after the loads land, store those rows into the pool.
template <int D>
struct NewRow {
  const f16* k;  // k_new row of (b, g)
  const f16* v;  // v_new row of (b, g)
  int pos;       // absolute key index of the new token (-1: none)
};

// Loads of one 16-key tile (V rows non-temporal, as load_pair); the lanes
// holding key nr.pos read the new rows.  Keys past nr.pos lie beyond the
// sequence (the new token is its last key), so their lanes read the new rows
// too instead of pool rows that would be masked anyway: a tail tile costs no
// HBM traffic beyond its valid rows (at 4097 attended keys the last tile
// holds the new token alone, and its wave would otherwise stream a whole
// extra tile).  With nr.pos < 0 (no append) every lane reads the pool.
template <int D>
__device__ __forceinline__ void load_tile_new(f16x8 (&k)[Geo<D>::KS],
                                              typename HVec<Geo<D>::NT>::type (&v)[4],
                                              const PagedSrc& src, TileLoc tl, int kt0,
                                              const NewRow<D>& nr, int r16, int grp) {
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  typedef typename HVec<NT>::type vrow_t;
  auto past = [&](int row) { return nr.pos >= 0 && kt0 + row >= nr.pos; };
  const f16* kp = past(r16) ? nr.k + 8 * grp : src.k_pool + tl.base + r16 * D + 8 * grp;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) k[ks] = *reinterpret_cast<const f16x8*>(kp + 32 * ks);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = 4 * grp + e;
    const f16* vp = past(row) ? nr.v + NT * r16 : src.v_pool + tl.base + row * D + NT * r16;
    v[e] = stream_load(reinterpret_cast<const vrow_t*>(vp));
  }
}

// Both tiles are always loaded (a step with one tile loads it twice and
// masks the copy, key0b = kNoKey), as load_pair does.
template <int D, bool kAppend>
__device__ __forceinline__ void load_pair_new(KVPair<D>& kv, const PagedSrc& src, TileLoc t0,
                                              TileLoc t1, int key0a, int key0b,
                                              const NewRow<D>& nr, int r16, int grp) {
  typedef typename HVec<Geo<D>::NT>::type vrow_t;
  typedef vrow_t vquad_t[4];
  if constexpr (!kAppend) {
    load_pair<D>(kv, src.k_pool, src.v_pool, t0, t1, r16, grp);
  } else {
    load_tile_new<D>(kv.k[0], *reinterpret_cast<vquad_t*>(&kv.v[0]), src, t0, key0a, nr, r16, grp);
    load_tile_new<D>(kv.k[1], *reinterpret_cast<vquad_t*>(&kv.v[4]), src, t1, key0b, nr, r16, grp);
  }
}

// Store the new token's rows (already in registers) into the pool.  The
// register arrays are only ever indexed with compile-time indices (a runtime
// index would move the whole pair to scratch memory).
template <int D>
__device__ __forceinline__ void store_new_row(const KVPair<D>& kv, const PagedSrc& src,
                                              TileLoc t0, TileLoc t1, int key0a, int key0b,
                                              int pos, int r16, int grp) {
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  typedef typename HVec<NT>::type vrow_t;
  const bool second = pos >= key0b;
  const int row = pos - (second ? key0b : key0a);
  const int64_t base = (second ? t1.base : t0.base) + (int64_t)row * D;
  f16* kpool = const_cast<f16*>(src.k_pool);
  f16* vpool = const_cast<f16*>(src.v_pool);
  if (r16 == row) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const f16x8 kk = second ? kv.k[1][ks] : kv.k[0][ks];
      *reinterpret_cast<f16x8*>(kpool + base + 8 * grp + 32 * ks) = kk;
    }
  }
  if ((row >> 2) == grp) {
    vrow_t vv = vrow_t{};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e == 4 * (int)second + (row & 3)) vv = kv.v[e];
    *reinterpret_cast<vrow_t*>(vpool + base + NT * r16) = vv;
  }
}

// RoPE of the Q / K operand dims a lane holds (dims 8*grp + 32*ks + j, j < 8):
// the partners i and i + D/2 of rotate_half sit in k-steps ks and ks + KS/2
// of the same lane, so no lane exchange is needed.
template <int D>
__device__ __forceinline__ void rope_lane(f16x8 (&x)[Geo<D>::KS], const f16x8 (&c)[Geo<D>::KS],
                                          const f16x8 (&s)[Geo<D>::KS]) {
  constexpr int H = Geo<D>::KS / 2;
#pragma unroll
  for (int ks = 0; ks < H; ++ks) rope8(x[ks], x[ks + H], c[ks], c[ks + H], s[ks], s[ks + H]);
}

// Rope mode: put the rotated K row of the new token (knew, held by every lane
// for its dims) into the lanes of its key in a loaded pair, replacing the
// unrotated row the tile load read from k_new.  pos must lie in the pair.
template <int D>
__device__ __forceinline__ void put_new_k(KVPair<D>& kv, int key0a, int key0b, int pos,
                                          const f16x8 (&knew)[Geo<D>::KS], int r16) {
  const bool second = pos >= key0b;
  const int row = pos - (second ? key0b : key0a);
  // selects, not branches: a conditional write into the register-staged pair
  // would make the compiler move the pair to scratch memory
  const bool in_a = r16 == row && !second;
  const bool in_b = r16 == row && second;
#pragma unroll
  for (int ks = 0; ks < Geo<D>::KS; ++ks) {
    kv.k[0][ks] = in_a ? knew[ks] : kv.k[0][ks];
    kv.k[1][ks] = in_b ? knew[ks] : kv.k[1][ks];
  }
}

// Split partials cross workgroups (and XCDs, each with its own L2): they are
// written and read only as agent-scope atomics (global_store / global_load /
// buffer accesses with sc1), coherent device-wide (arrive_last).
__device__ __forceinline__ void partial_store(float* ptr, float v) { agent_store(ptr, v); }
__device__ __forceinline__ float partial_load(const float* ptr) { return agent_load(ptr); }

constexpr int kMaxSplits = 64;

// Where the split partials of one (sequence, kv head) live: the row of (head
// h of the group, split s) is base + h * hs + s * ss, and the group's G * S
// rows are contiguous from base.  Unplanned launches keep (b, head, split)
// order (hs = S, ss = 1); planned ones index by workgroup, (w_first + s,
// head) (hs = 1, ss = G), so the partials are sized by the grid.
struct PartRows {
  int64_t base;
  int hs, ss;
  __device__ __forceinline__ int rel(int h, int s) const { return h * hs + s * ss; }
};

// A step's plan (cie_paged_decode_plan): per workgroup kPlanDescWords int32
// — b (-1: idle), g, split, S, slot, L, pos (-1: no append), w_first (the
// group's first workgroup) — then per workgroup and wave the page ids of the
// wave's first 64 tiles.
constexpr int kPlanDescWords = 8;
constexpr int kPlanWaves = 4;

template <int D, int NTHREADS>
__device__ __forceinline__ void merge_splits(const DecodeParams& p, const PartRows& prow, int b,
                                             int g, int n_states, int tid);

// Profiling builds only (-DCIE_DECODE_TRACE): phase boundaries
// (s_memrealtime) are stamped into LDS — LDS writes do not count in vmcnt, so
// the stamps do not lengthen the waits on the K/V loads — and each workgroup
// copies its 24 stamps to the buffer named by cie_decode_trace_buffer()
// (exported by such builds alone) when it exits.
#ifdef CIE_DECODE_TRACE
constexpr int kTraceSlots = 24;
__device__ uint64_t* g_decode_trace;
#define DECODE_TRACE_LANE0(k, v)                              \
  do {                                                        \
    if ((threadIdx.x & (kWave - 1)) == 0) sm_trace[(k)] = (v); \
  } while (0)
#if CIE_DECODE_TRACE == 2
// per-wave stamps only (the single-thread phase stamps off, start excepted)
#define DECODE_TRACE(k, v)                                 \
  do {                                                     \
    if ((k) == 0 || (k) == 5 || (k) == 6)                  \
      if (threadIdx.x == 0) sm_trace[(k)] = (v);           \
  } while (0)
#else
#define DECODE_TRACE(k, v)                  \
  do {                                      \
    if (threadIdx.x == 0) sm_trace[(k)] = (v); \
  } while (0)
#endif
#define DECODE_TRACE_DUMP()                                                                          \
  do {                                                                                               \
    __syncthreads();                                                                                 \
    if (threadIdx.x < kTraceSlots && g_decode_trace != nullptr)                                      \
      g_decode_trace[(int64_t)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)) *    \
                         kTraceSlots + threadIdx.x] = sm_trace[threadIdx.x];                         \
  } while (0)
#else
#define DECODE_TRACE_LANE0(k, v) \
  do {                           \
  } while (0)
#define DECODE_TRACE(k, v) \
  do {                     \
  } while (0)
#define DECODE_TRACE_DUMP() \
  do {                      \
  } while (0)
#endif

// At D = 64 two waves per SIMD must fit (256 registers a wave), so grids of
// up to two workgroups per CU stay resident in one round.  The leading
// arguments repeat p.slot_ids, p.plan and p.n_wg, the fields the start's
// first load is indexed by: as scalar arguments ahead of the struct they are
// preloaded into SGPRs (the build's kernel-argument preload count), so that
// load goes out without waiting for the kernel-argument load (-0.1 to
// -0.4 us per call).
template <int D, int WAVES, bool kAppend, bool kRope, bool kPlanned>
__global__ __launch_bounds__(WAVES * kWave) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1)))
void decode_kernel(const int64_t* __restrict__ a_slot_ids, const int32_t* __restrict__ a_plan,
                   int32_t a_n_wg, DecodeParams p) {
  static_assert(kAppend || !kRope, "rope mode appends");
  static_assert(!kPlanned || WAVES == kPlanWaves, "a plan holds the page ids of kPlanWaves waves");
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  __shared__ float sm_m[WAVES][16];
  __shared__ float sm_l[WAVES][16];
  // rows padded to keep 16-byte alignment for the vector reads of the fold
  __shared__ f32x4 sm_acc[WAVES][16][D / 4 + 1];
  __shared__ int sm_last;
#ifdef CIE_DECODE_TRACE
  __shared__ uint64_t sm_trace[kTraceSlots];
  if (threadIdx.x < kTraceSlots) sm_trace[threadIdx.x] = 0;
  __syncthreads();
#endif

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r16 = lane & 15;
  const int grp = lane >> 4;
  const int tpp = p.page_size >> 4;  // 16-key tiles per page
  const int row_tiles = p.bt_width * tpp;
  // One page id per lane: a wave of up to 64 tiles (its odd last tile
  // included) never waits on another block-table load before streaming.
  constexpr int kSpecTiles = kWave;

  DECODE_TRACE(0, __builtin_amdgcn_s_memrealtime());
  DECODE_TRACE(5, (uint64_t)__builtin_amdgcn_s_getreg(0xF804));  // HW_ID
  DECODE_TRACE(6, (uint64_t)__builtin_amdgcn_s_getreg(0xF814));  // XCC_ID

  // The workgroup's work: split `split` of the S of (sequence b, kv head g),
  // the slot, the L keys to attend (append mode: pos + 1, the new token at
  // pos), and the page ids of this wave's first kSpecTiles tiles, one per lane.
  // Wave gw of the TW = S * WAVES waves of the (sequence, kv head) takes key
  // tiles gw, gw + TW, gw + 2*TW, ...; its k-th tile's page id is held by lane
  // k (read back with readlane), so a step never waits on a block-table load.
  int split, g, b, S, L, pos = -1, w_first = 0, pages = 0;
  int64_t slot;
  f16x8 qop[1][KS];
  f16x8 cs[KS], sn[KS], knew[KS];
  // Q^T operand (column r16 = head g*G + r16, zero past the group), and in
  // rope mode the new token's cos / sin rows and unrotated K row.
  auto load_q = [&]() {
    const f16* qrow = p.q + (int64_t)b * p.q_row_stride + (int64_t)(g * p.G + r16) * D + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qop[0][ks] = (r16 < p.G) ? *reinterpret_cast<const f16x8*>(qrow + 32 * ks) : f16x8{};
    if constexpr (kRope) {
      const f16* crow = p.cos + (int64_t)b * p.cs_stride + 8 * grp;
      const f16* srow = p.sin + (int64_t)b * p.cs_stride + 8 * grp;
      const f16* krow = p.k_new + (int64_t)b * p.k_tok_stride + (int64_t)g * p.k_head_stride + 8 * grp;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        cs[ks] = *reinterpret_cast<const f16x8*>(crow + 32 * ks);
        sn[ks] = *reinterpret_cast<const f16x8*>(srow + 32 * ks);
        knew[ks] = *reinterpret_cast<const f16x8*>(krow + 32 * ks);
      }
    }
  };
  if constexpr (kPlanned) {
    // A step's plan (cie_paged_decode_plan) holds this workgroup's descriptor
    // and its waves' page ids: one memory round trip, after which Q and the
    // first K/V tiles go out together.  Its indices were checked when it was
    // made.
    const int w = blockIdx.x;
    const int32_t* d = a_plan + (int64_t)w * kPlanDescWords;
    pages = a_plan[(int64_t)a_n_wg * kPlanDescWords + ((int64_t)w * kPlanWaves + wave) * kWave + lane];
    b = d[0];
    if (b < 0) return;  // a workgroup the plan left idle (uniform)
    g = d[1];
    split = d[2];
    S = d[3];
    slot = d[4];
    L = d[5];
    pos = d[6];
    w_first = d[7];
    load_q();
  } else {
    split = blockIdx.x;
    g = blockIdx.y;
    b = blockIdx.z;
    S = p.n_splits;
    // The first kSpecTiles page ids are fetched as soon as the slot is known,
    // in parallel with the length, which in append mode is itself a load
    // indexed by the slot.  Every load of the start goes out before any
    // check: a check's error store (set_err) may alias later loads as far as
    // the compiler knows, so a check placed between two loads makes the
    // second wait for the first's data.  Issued together, the first tiles'
    // page ids, the length and Q take one memory round trip.
    const int gw0 = split * WAVES + wave;
    slot = a_slot_ids[b];
    const bool slot_ok = slot >= 0 && slot < p.n_slots;
    if (!slot_ok) {
      set_err(p.err, CIE_ERRBIT_PAGE);
      slot = 0;
    }
    const int64_t* row = p.block_table + slot * p.bt_stride;
    const int t_spec = gw0 + lane * S * WAVES;
    const int64_t page_spec = (lane < kSpecTiles && t_spec < row_tiles) ? row[t_spec / tpp] : 0;
    const int64_t len_raw = kAppend ? p.lens[slot] : p.lens[b];
    load_q();
    const int64_t cap = (int64_t)row_tiles * 16;
    if constexpr (kAppend) {
      const int64_t prior = len_raw;
      if (!slot_ok || prior < 0 || prior + 1 > cap) {
        if (slot_ok) set_err(p.err, CIE_ERRBIT_LEN);
        L = 0;
      } else {
        pos = (int)prior;
        L = pos + 1;
      }
    } else {
      int64_t len = len_raw;
      if (len < 0 || len > cap) {
        set_err(p.err, CIE_ERRBIT_LEN);
        len = len < 0 ? 0 : cap;
      }
      L = slot_ok ? (int)len : 0;
    }
    // Speculatively fetched page ids of tiles past the sequence are never
    // used (and never reported: the row may hold anything there).
    if (lane < kSpecTiles && t_spec < ((L + 15) >> 4)) {
      int64_t page = page_spec;
      if (page < 0 || page >= p.n_pages) {
        set_err(p.err, CIE_ERRBIT_PAGE);
        page = 0;
      }
      pages = (int)page;
    }
  }
  const int TW = S * WAVES;
  const int gw = split * WAVES + wave;
  const int64_t* bt_row = p.block_table + slot * p.bt_stride;
  auto lane_page = [&](int k) -> int {  // page id of this wave's k-th tile
    const int t = gw + k * TW;
    if (t >= row_tiles) return 0;
    int64_t page = bt_row[t / tpp];
    if (page < 0 || page >= p.n_pages) {
      set_err(p.err, CIE_ERRBIT_PAGE);
      page = 0;
    }
    return (int)page;
  };
  const int n_tiles = (L + 15) >> 4;
  const int n_mine = n_tiles > gw ? (n_tiles - gw + TW - 1) / TW : 0;
  // where this workgroup's partial rows live (see PartRows)
  const PartRows prow = kPlanned ? PartRows{(int64_t)w_first * p.G, 1, p.G}
                                 : PartRows{((int64_t)b * p.H_q + g * p.G) * S, S, 1};

  const PagedSrc src{p.k_pool,  p.v_pool,  bt_row, (int64_t)g * p.pool_head_stride,
                     p.pool_page_stride, p.n_pages, p.page_size, p.err};
  NewRow<D> nr{nullptr, nullptr, -1};
  if constexpr (kAppend) {
    nr.k = p.k_new + (int64_t)b * p.k_tok_stride + (int64_t)g * p.k_head_stride;
    nr.v = p.v_new + (int64_t)b * p.v_tok_stride + (int64_t)g * p.v_head_stride;
    nr.pos = pos;
  }
  // Rope mode: q and the new token's K row (every lane its dims, loaded with
  // the start's other loads, for the lanes of that key to take once its tile
  // is loaded) are rotated once the first K/V loads have been issued, so the
  // wait for q, cos and sin and the rotation do not hold those loads back
  // (rotating first cost ~0.6 us per call at config 2).
  auto rotate = [&]() {
    if constexpr (kRope) {
      rope_lane<D>(qop[0], cs, sn);
      rope_lane<D>(knew, cs, sn);
    }
  };

  DECODE_TRACE(1, __builtin_amdgcn_s_memrealtime());
  DECODE_TRACE(7, (uint64_t)n_mine);
  SoftmaxAcc<D, 1> st;
  st.init();
  const int lim[1] = {L};

  // A wave with an odd tile count takes its last tile out of the two-tile
  // steps: that tile's loads go out now, ahead of the first step's, and it is
  // attended right after the first step (whose wait covers it: loads complete
  // in issue order).  When the tiles of a (sequence, kv head) do not divide
  // evenly over its waves, the waves holding one tile more would otherwise run
  // one more dependent step than all the others, and every wave of the call
  // would wait for them.  In append mode the new token's rows, if they sit in
  // that tile, are stored to the pool after the loop: a store inside the loop
  // would make every later wait there cover the store's completion too.
  typedef typename HVec<NT>::type vrow_t;
  typedef vrow_t vquad_t[4];
  const bool odd = n_mine & 1;
  const int n_main = n_mine - (odd ? 1 : 0);
  KVPair<D> xt;
  int xkey = kNoKey;
  TileLoc xloc{0};
  if (odd) {
    const int kx = n_mine - 1;
    const int tx = gw + kx * TW;
    const int px = kx < kSpecTiles ? __builtin_amdgcn_readlane(pages, kx) : uniform(lane_page(kx));
    xloc = TileLoc{(int64_t)px * src.page_stride + src.head_off + (int64_t)((tx % tpp) * 16) * D};
    xkey = tx * 16;
    load_tile_new<D>(xt.k[0], *reinterpret_cast<vquad_t*>(&xt.v[0]), src, xloc, xkey, nr, r16, grp);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) xt.k[1][ks] = f16x8{};
#pragma unroll
    for (int e = 4; e < 8; ++e) xt.v[e] = vrow_t{};
  }
  auto attend_odd = [&]() {
    if (xkey + 16 >= L) zero_tail_rows<D>(xt, xkey, kNoKey, L, grp);
    if constexpr (kRope) {
      if (pos >= xkey && pos < xkey + 16) put_new_k<D>(xt, xkey, kNoKey, pos, knew, r16);
    }
    attend_pair<D, 1>(st, xt, QRegs<D, 1>{qop}, xkey, kNoKey, lim, L, p.scale_log2, grp);
  };

  for (int c0 = 0; c0 < n_main; c0 += kWave) {
    // this chunk's page ids: lanes k = c0 + lane (the first chunk's first
    // kSpecTiles are already in flight)
    if (c0 > 0 || n_main > kSpecTiles) {
      const int k = c0 + lane;
      if (c0 > 0 || lane >= kSpecTiles) pages = k < n_main ? lane_page(k) : 0;
    }
    const int n_chunk = min(kWave, n_main - c0);
    const int n_pairs = (n_chunk + 1) >> 1;
    // Ring of kPF + 1 register-staged pairs: pair j's loads are issued kPF
    // steps before its math, so up to kPF pairs of loads are in flight.
    // Every iteration issues exactly one pair, so the wait before a pair's
    // math covers that pair's loads only.  Past the end the pair it issues
    // reads cached lines — the new token's row (append mode), or the last
    // pair's K lines for both K and V — because re-read V rows, loaded
    // non-temporal, would come from HBM again and hold up the wave's final
    // vmcnt(0) before its arrival atomic.
    constexpr int kPF = CIE_DECODE_PF;
    KVPair<D> ring[kPF + 1];
    TileLoc loc[kPF + 1][2];
    int keya[kPF + 1], keyb[kPF + 1];
    auto issue = [&](int slot_i, int j) {
      const bool real = j < n_pairs;
      const f16* vpool = real ? src.v_pool : src.k_pool;
      j = min(j, n_pairs - 1);
      const int ka = 2 * j;                // chunk-local index of tile A
      const bool two = ka + 1 < n_chunk;
      const int ta = gw + (c0 + ka) * TW;  // tile ids
      const int tb = two ? ta + TW : ta;
      const int pa = __builtin_amdgcn_readlane(pages, ka);
      const int pb = two ? __builtin_amdgcn_readlane(pages, ka + 1) : pa;
      loc[slot_i][0] = TileLoc{(int64_t)pa * src.page_stride + src.head_off +
                               (int64_t)((ta % tpp) * 16) * D};
      loc[slot_i][1] = TileLoc{(int64_t)pb * src.page_stride + src.head_off +
                               (int64_t)((tb % tpp) * 16) * D};
      keya[slot_i] = ta * 16;
      keyb[slot_i] = two ? tb * 16 : kNoKey;
      if constexpr (kAppend)
        // past the end every lane reads the new token's row (cached), as
        // the lanes of keys at or past pos do: no second address set
        load_pair_new<D, kAppend>(ring[slot_i], src, loc[slot_i][0], loc[slot_i][1],
                                  real ? keya[slot_i] : pos, real ? keyb[slot_i] : pos, nr, r16, grp);
      else
        load_pair<D>(ring[slot_i], src.k_pool, vpool, loc[slot_i][0], loc[slot_i][1], r16, grp);
    };
#pragma unroll
    for (int j = 0; j < kPF; ++j) issue(j, j);
    if (c0 == 0) rotate();
    for (int j0 = 0; j0 < n_pairs; j0 += kPF + 1) {
#pragma unroll
      for (int u = 0; u <= kPF; ++u) {
        const int j = j0 + u;
        issue((u + kPF) % (kPF + 1), j + kPF);
        if (j < n_pairs) {
          KVPair<D>& cur = ring[u];
          const int ka = keya[u], kb = keyb[u];
          const int last_key = (kb == kNoKey ? ka : kb) + 16;
          if (last_key >= L) {  // this pair holds the sequence's last key
            zero_tail_rows<D>(cur, ka, kb, L, grp);
            if constexpr (kAppend) {
              // the new token is the sequence's last key: it sits in this pair
              if (pos >= ka) {
                if constexpr (kRope) put_new_k<D>(cur, ka, kb, pos, knew, r16);
                store_new_row<D>(cur, src, loc[u][0], loc[u][1], ka, kb, pos, r16, grp);
              }
            }
          }
          attend_pair<D, 1>(st, cur, QRegs<D, 1>{qop}, ka, kb, lim, L, p.scale_log2, grp);
        }
        if (c0 == 0 && j == 0) DECODE_TRACE_LANE0(20 + wave, __builtin_amdgcn_s_memrealtime());
        if (odd && c0 == 0 && j == 0) attend_odd();
      }
    }
  }
  // Append mode: if the new token sits in this wave's odd tile, its rows go
  // to the pool only after the workgroup's arrival (store_odd below): issued
  // here, their completion would join the wait for the partial stores that
  // the arrival atomic follows (0.1 us per call at config 2).  Rope mode
  // stores them here (deferred, its build ran 0.2 us slower).
  auto store_odd = [&]() {
    if constexpr (kAppend) {
      if (odd && pos >= xkey && pos < xkey + 16)
        store_new_row<D>(xt, src, xloc, xloc, xkey, kNoKey, pos, r16, grp);
    }
  };
  if constexpr (kRope) {
    if (odd) {
      if (n_main == 0) {
        rotate();
        attend_odd();
      }
      if (pos >= xkey && pos < xkey + 16)
        store_new_row<D>(xt, src, xloc, xloc, xkey, kNoKey, pos, r16, grp);
    }
  } else if (odd && n_main == 0) {
    attend_odd();
  }

  DECODE_TRACE(2, __builtin_amdgcn_s_memrealtime());
  DECODE_TRACE_LANE0(16 + wave, __builtin_amdgcn_s_memrealtime());
  // Fold the waves of this workgroup.  Lane (r16, grp) holds dims
  // NT*(4*grp + r) + nt of column r16: for each r, NT consecutive dims, written
  // as NT/4 16-byte vectors.  One thread then folds 4 dims of one head.
  if (grp == 0) {
    sm_m[wave][r16] = st.m[0];
    sm_l[wave][r16] = st.l(0);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int n4 = 0; n4 < NT / 4; ++n4)
      sm_acc[wave][r16][(NT * (4 * grp + r)) / 4 + n4] =
          f32x4{st.acc[0][4 * n4][r], st.acc[0][4 * n4 + 1][r], st.acc[0][4 * n4 + 2][r],
                st.acc[0][4 * n4 + 3][r]};
  __syncthreads();
  DECODE_TRACE(8, __builtin_amdgcn_s_memrealtime());

  constexpr int D4 = D / 4;
  const __amdgpu_buffer_rsrc_t racc =
      coherent_rsrc(p.part_acc + prow.base * D, (uint32_t)(p.G * S * D * sizeof(float)));
  for (int it = threadIdx.x; it < p.G * D4; it += WAVES * kWave) {
    const int h = it / D4;
    const int d4 = it - h * D4;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][h]);
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float mw = sm_m[w][h];
      // a wave that saw no key has m = -inf, l = 0, acc = 0
      const float a = mw == kNegInf ? 0.f : fast_exp2(mw - M);
      num += a * sm_acc[w][h][d4];
      den += a * sm_l[w][h];
    }
    if (S == 1) {
      const bool none = M == kNegInf || den == 0.f;
      f16x4 o4;
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = (f16)(none ? 0.f : num[i] / den);
      *reinterpret_cast<f16x4*>(p.o + ((int64_t)b * p.H_q + g * p.G + h) * D + 4 * d4) = o4;
    } else {
      const int row = prow.rel(h, split);  // within the group's rows
      agent_store4(racc, (uint32_t)((row * D + 4 * d4) * sizeof(float)), num);
      if (d4 == 0) {
        partial_store(&p.part_m[prow.base + row], M);
        partial_store(&p.part_l[prow.base + row], den);
      }
    }
  }
  DECODE_TRACE(9, __builtin_amdgcn_s_memrealtime());
  if (S == 1) {
    if constexpr (!kRope) store_odd();
    DECODE_TRACE_DUMP();
    return;
  }

  // The last workgroup of this (sequence, kv head) to arrive merges the splits.
  int32_t* const arrival = p.counters + b * p.H_kv + g;
  const bool last = arrive_last(arrival, (int64_t)p.B * p.H_kv, S, &sm_last, p.err);
  DECODE_TRACE(10, __builtin_amdgcn_s_memrealtime());
  if constexpr (!kRope) store_odd();
  if (!last) {
    DECODE_TRACE_DUMP();
    return;
  }
  merge_splits<D, WAVES * kWave>(p, prow, b, g, S, threadIdx.x);
  if (threadIdx.x == 0) counter_reset(arrival);
  DECODE_TRACE(4, __builtin_amdgcn_s_memrealtime());
  DECODE_TRACE_DUMP();
}

// Combine the S partial states of every head of (b, g) into o.  A thread
// owns 4 dims of one head and takes the splits in groups of kMergeGroup: the m, l
// and acc loads of a group are all issued before any is used (one memory round
// trip per group), and a running log-sum-exp carries across groups.  For
// S <= kMergeGroup the arithmetic is the plain max-then-sum of
// kernels/decode_attention.py:243-264.
constexpr int kMergeGroup = 8;

template <int D, int NTHREADS>
__device__ __forceinline__ void merge_splits(const DecodeParams& p, const PartRows& prow, int b,
                                             int g, int n_states, int tid) {
  constexpr int D4 = D / 4;
  const int S = n_states;
  const __amdgpu_buffer_rsrc_t racc =
      coherent_rsrc(p.part_acc + prow.base * D, (uint32_t)(p.G * S * D * sizeof(float)));
  for (int it = tid; it < p.G * D4; it += NTHREADS) {
    const int h = it / D4;
    const int d4 = it - h * D4;
    float M = kNegInf, den = 0.f;
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < S; s0 += kMergeGroup) {
      float ms[kMergeGroup], ls[kMergeGroup];
      f32x4 as[kMergeGroup];
#pragma unroll
      for (int u = 0; u < kMergeGroup; ++u) {
        ms[u] = kNegInf;
        ls[u] = 0.f;
        as[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (s0 + u < S) {
          const int row = prow.rel(h, s0 + u);
          ms[u] = partial_load(&p.part_m[prow.base + row]);
          ls[u] = partial_load(&p.part_l[prow.base + row]);
          as[u] = agent_load4(racc, (uint32_t)((row * D + 4 * d4) * sizeof(float)));
        }
      }
      float Mn = M;
#pragma unroll
      for (int u = 0; u < kMergeGroup; ++u) Mn = fmaxf(Mn, ms[u]);
      if (Mn == kNegInf) continue;  // no split of this group saw a key
      // rescale what earlier groups summed (exp2(-inf) = 0 while M is unset)
      const float c = fast_exp2(M - Mn);
      num *= c;
      den *= c;
#pragma unroll
      for (int u = 0; u < kMergeGroup; ++u) {
        const float a = ms[u] == kNegInf ? 0.f : fast_exp2(ms[u] - Mn);
        num += a * as[u];
        den += a * ls[u];
      }
      M = Mn;
    }
    const bool none = M == kNegInf || den == 0.f;
    f16x4 o4;
#pragma unroll
    for (int i = 0; i < 4; ++i) o4[i] = (f16)(none ? 0.f : num[i] / den);
    *reinterpret_cast<f16x4*>(p.o + ((int64_t)b * p.H_q + g * p.G + h) * D + 4 * d4) = o4;
  }
}

// ---------------------------------------------------------------------------
// A decode step's plan.  The slot ids, lengths and block-table rows a decode
// reads are the same for every layer of a step (the lengths advance after
// the last layer), so one small launch per step works out what each layer's
// launch would otherwise redo: every sequence's attended length, how many
// workgroups (splits) each (sequence, kv head) gets, and each workgroup's
// page ids.  A planned decode launch then needs one memory round trip (its
// descriptor and its waves' page ids) before its first K/V loads, where an
// unplanned one needs two (slot id, then page ids and length).
//
// Splits are balanced by length: tau, the smallest tile count per split for
// which sum_b max(1, ceil(tiles_b / tau)) splits (at most kMaxSplits each)
// fit the grid's n_wg / H_kv workgroups per kv head, gives sequence b
// ceil(tiles_b / tau) splits, so the longest sequences no longer set the call
// when lengths differ.  Equal lengths get equal splits (the unplanned deal).
// Every workgroup of the plan launch redoes the balance (a few hundred
// sequences at most, LDS only) and then writes its own descriptor and page
// ids: no workgroup waits on another.
constexpr int kPlanMaxSeqs = 1024;
constexpr int kPlanThreads = kPlanWaves * kWave;

struct PlanParams {
  int32_t* plan;
  const int64_t* lens;  // append: (n_slots,) prior length per slot; plain: (B,) attended
  const int64_t* slot_ids;
  const int64_t* block_table;
  int64_t bt_stride, n_pages;
  int32_t B, H_kv, page_size, bt_width, n_slots, n_wg, append;
  int32_t* err;
};

__device__ __forceinline__ int plan_block_sum(int x, int* sm_red) {
  for (int off = 1; off < kWave; off <<= 1) x += __shfl_xor(x, off, kWave);
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) sm_red[threadIdx.x / kWave] = x;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < kPlanWaves; ++w) t += sm_red[w];
  return t;
}

// A sequence's attended length as the decode kernel derives it (with its
// index checks; `report` lets one workgroup of the plan report errors).
__device__ __forceinline__ int plan_seq(const PlanParams& p, int bb, int64_t cap, bool report,
                                        int* slot_out) {
  int64_t slot = p.slot_ids[bb];
  const bool slot_ok = slot >= 0 && slot < p.n_slots;
  if (!slot_ok) {
    if (report) set_err(p.err, CIE_ERRBIT_PAGE);
    slot = 0;
  }
  const int64_t len = p.append ? p.lens[slot] : p.lens[bb];
  int L;
  if (p.append) {
    if (!slot_ok || len < 0 || len + 1 > cap) {
      if (slot_ok && report) set_err(p.err, CIE_ERRBIT_LEN);
      L = 0;
    } else {
      L = (int)len + 1;
    }
  } else {
    int64_t l = len;
    if (l < 0 || l > cap) {
      if (report) set_err(p.err, CIE_ERRBIT_LEN);
      l = l < 0 ? 0 : cap;
    }
    L = slot_ok ? (int)l : 0;
  }
  *slot_out = (int)slot;
  return L;
}

__device__ __forceinline__ int plan_splits(int nt, int tau) {
  return min(kMaxSplits, max(1, (nt + tau - 1) / tau));
}

// Writes workgroup w's descriptor (desc[0..7], lanes 0..7 of one wave) and the
// page ids of wave j (one per lane k) of that workgroup.
__device__ __forceinline__ void plan_write(const PlanParams& p, int w, int j, int lane, int bb,
                                           int nt, int S, int w0, int slot, int L, int tpp) {
  const int g = (w - w0) / S;
  const int split = (w - w0) - g * S;
  if (j == 0 && lane < kPlanDescWords) {
    const int v[kPlanDescWords] = {bb, g, split, S, slot, L, p.append && L > 0 ? L - 1 : -1,
                                   w0 + g * S};
    int x = v[0];
#pragma unroll
    for (int i = 1; i < kPlanDescWords; ++i) x = lane == i ? v[i] : x;
    p.plan[(int64_t)w * kPlanDescWords + lane] = x;
  }
  // wave j of split s deals tiles (s * kPlanWaves + j) + k * S * kPlanWaves
  const int t = split * kPlanWaves + j + lane * S * kPlanWaves;
  int page = 0;
  if (t < nt) {
    int64_t pg = p.block_table[(int64_t)slot * p.bt_stride + t / tpp];
    if (pg < 0 || pg >= p.n_pages) {
      set_err(p.err, CIE_ERRBIT_PAGE);
      pg = 0;
    }
    page = (int)pg;
  }
  p.plan[(int64_t)p.n_wg * kPlanDescWords + ((int64_t)w * kPlanWaves + j) * kWave + lane] = page;
}

// Batches of up to kWave sequences: every wave plans alone, a sequence per
// lane (shuffle reductions and scan, no LDS, no barrier).  The search for tau
// starts at its lower bound ceil(sum of tiles / workgroups per kv head): a
// split count sum over sequences is at least tiles / tau, so no smaller tau
// fits; with equal lengths the bound itself fits.
__device__ __forceinline__ void plan_wave(const PlanParams& p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int j = threadIdx.x / kWave;
  const int B = p.B;
  const int tpp = p.page_size >> 4;
  const int64_t cap = (int64_t)p.bt_width * tpp * 16;
  int slot = 0, L = 0;
  if (lane < B) L = plan_seq(p, lane, cap, blockIdx.x == 0 && j == 0, &slot);
  const int nt = (L + 15) >> 4;
  int total = lane < B ? nt : 0, hi = nt;
  for (int off = 1; off < kWave; off <<= 1) {
    total += __shfl_xor(total, off, kWave);
    hi = max(hi, __shfl_xor(hi, off, kWave));
  }
  const int n_ph = p.n_wg / p.H_kv;
  auto fits = [&](int tau) {
    int c = lane < B ? plan_splits(nt, tau) : 0;
    for (int off = 1; off < kWave; off <<= 1) c += __shfl_xor(c, off, kWave);
    return c <= n_ph;
  };
  int lo = max(1, (total + n_ph - 1) / n_ph);
  hi = max(hi, lo);
  if (!fits(lo)) {  // binary search in (lo, hi]; hi always fits (one split each)
    while (lo + 1 < hi) {
      const int mid = (lo + hi) >> 1;
      if (fits(mid))
        hi = mid;
      else
        lo = mid;
    }
    lo = hi;
  }
  const int tau = lo;
  // first workgroup of each sequence: exclusive scan of H_kv * splits
  const int S_b = lane < B ? plan_splits(nt, tau) : 0;
  int x = p.H_kv * S_b;
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  const int w0_b = x - p.H_kv * S_b;
  const int used = __shfl(x, kWave - 1, kWave);
  const int w = blockIdx.x;
  if (w >= used) {
    if (j == 0 && lane == 0) p.plan[(int64_t)w * kPlanDescWords] = -1;
    return;
  }
  // my sequence: the last lane whose first workgroup is at or before w
  const uint64_t at_or_before = __ballot(lane < B && w0_b <= w);
  const int bb = __popcll(at_or_before) - 1;
  plan_write(p, w, j, lane, bb, __shfl(nt, bb, kWave), __shfl(S_b, bb, kWave), __shfl(w0_b, bb, kWave),
             __shfl(slot, bb, kWave), __shfl(L, bb, kWave), tpp);
}

__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(PlanParams p) {
  if (p.B <= kWave) {
    plan_wave(p);
    return;
  }
  __shared__ int sm_nt[kPlanMaxSeqs];       // key tiles of sequence b (L + 15) / 16
  __shared__ int sm_len[kPlanMaxSeqs];      // attended keys L
  __shared__ int sm_slot[kPlanMaxSeqs];
  __shared__ int sm_w0[kPlanMaxSeqs + 1];   // first workgroup of sequence b
  __shared__ int sm_red[kPlanWaves];
  const int tid = threadIdx.x;
  const int B = p.B;
  const int tpp = p.page_size >> 4;
  const int row_tiles = p.bt_width * tpp;
  const int64_t cap = (int64_t)row_tiles * 16;
  // index errors are reported once, by workgroup 0 (every workgroup sees them)
  const bool report = blockIdx.x == 0;

  // 1. every sequence's slot and attended length, with the decode kernel's checks
  int my_max = 0;
  for (int bb = tid; bb < B; bb += kPlanThreads) {
    int slot;
    const int L = plan_seq(p, bb, cap, report, &slot);
    const int nt = (L + 15) >> 4;
    sm_nt[bb] = nt;
    sm_len[bb] = L;
    sm_slot[bb] = slot;
    my_max = max(my_max, nt);
  }
  for (int off = 1; off < kWave; off <<= 1) my_max = max(my_max, __shfl_xor(my_max, off, kWave));
  __syncthreads();
  if ((tid & (kWave - 1)) == 0) sm_red[tid / kWave] = my_max;
  __syncthreads();
  int hi = 1;
#pragma unroll
  for (int w = 0; w < kPlanWaves; ++w) hi = max(hi, sm_red[w]);

  // 2. the smallest tiles-per-split tau whose splits fit n_wg / H_kv per kv head
  const int n_ph = p.n_wg / p.H_kv;
  auto splits_of = [](int nt, int tau) { return plan_splits(nt, tau); };
  int lo = 1;
  while (lo < hi) {  // uniform: every thread holds the same bounds
    const int mid = (lo + hi) >> 1;
    int c = 0;
    for (int bb = tid; bb < B; bb += kPlanThreads) c += splits_of(sm_nt[bb], mid);
    if (plan_block_sum(c, sm_red) <= n_ph)
      hi = mid;
    else
      lo = mid + 1;
  }
  const int tau = lo;

  // 3. first workgroup of each sequence: exclusive prefix of H_kv * splits,
  // four consecutive sequences per thread
  {
    int v[4], run = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int bb = 4 * tid + u;
      v[u] = bb < B ? p.H_kv * splits_of(sm_nt[bb], tau) : 0;
      run += v[u];
    }
    // inclusive scan of run over the block
    int x = run;
    const int lane = tid & (kWave - 1);
    for (int off = 1; off < kWave; off <<= 1) {
      const int y = __shfl_up(x, off, kWave);
      if (lane >= off) x += y;
    }
    __syncthreads();
    if (lane == kWave - 1) sm_red[tid / kWave] = x;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < tid / kWave; ++w) base += sm_red[w];
    int e = base + x - run;  // exclusive prefix of this thread's first sequence
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int bb = 4 * tid + u;
      if (bb < B) sm_w0[bb] = e;
      e += v[u];
    }
    if (tid == kPlanThreads - 1) sm_w0[B] = base + x;  // total (sequences past B add 0)
  }
  __syncthreads();

  // 4. this workgroup's entry
  const int w = blockIdx.x;
  int32_t* const desc = p.plan + (int64_t)w * kPlanDescWords;
  if (w >= sm_w0[B]) {  // idle: the grid has more workgroups than the balance uses
    if (tid == 0) desc[0] = -1;
    return;
  }
  int lo_b = 0, hi_b = B - 1;  // the sequence with sm_w0[b] <= w < sm_w0[b + 1]
  while (lo_b < hi_b) {
    const int mid = (lo_b + hi_b + 1) >> 1;
    if (sm_w0[mid] <= w)
      lo_b = mid;
    else
      hi_b = mid - 1;
  }
  const int bb = lo_b;
  plan_write(p, w, tid / kWave, tid & (kWave - 1), bb, sm_nt[bb], splits_of(sm_nt[bb], tau), sm_w0[bb],
             sm_slot[bb], sm_len[bb], tpp);
}

// Waves per workgroup: four, one per SIMD.  With the non-temporal K/V loads
// a 4-wave workgroup per CU streams faster than an 8-wave one (config 2:
// 16.99 vs 18.08 us per call): the second wave per SIMD only queued more
// loads behind the first's and doubled the fold.  At D = 64 the kernel fits
// two waves per SIMD, so a grid of more workgroups than CUs (config 4: 512)
// is still resident in one round, two workgroups per CU.  D = 128 needs twice
// the registers (one wave per SIMD).  Variant builds with more waves halve
// them for such grids, so those also stay resident in one round.
template <int D>
constexpr int decode_waves() {
  return D <= 64 ? CIE_DECODE_WAVES : (CIE_DECODE_WAVES > 4 ? 4 : CIE_DECODE_WAVES);
}

static int device_cus() {
  constexpr int kMaxDevices = 64;
  static int cus[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

template <int D, int W, bool kAppend, bool kRope>
static int launch_decode_waves(const DecodeParams& p, hipStream_t stream) {
  dim3 grid(p.n_splits, p.H_kv, p.B);
  hipLaunchKernelGGL((decode_kernel<D, W, kAppend, kRope, false>), grid, dim3(W * kWave), 0, stream,
                     p.slot_ids, p.plan, p.n_wg, p);
  return (int)hipGetLastError();
}

template <int D, bool kAppend, bool kRope, bool kPlanned>
static int launch_decode(const DecodeParams& p, hipStream_t stream) {
  if constexpr (kPlanned) {  // one workgroup per plan entry, kPlanWaves waves each
    hipLaunchKernelGGL((decode_kernel<D, kPlanWaves, kAppend, kRope, true>), dim3(p.n_wg),
                       dim3(kPlanWaves * kWave), 0, stream, p.slot_ids, p.plan, p.n_wg, p);
    return (int)hipGetLastError();
  } else {
    constexpr int W = decode_waves<D>();
    constexpr int Wh = W > 4 ? W / 2 : W;
    const int64_t n_wg = (int64_t)p.n_splits * p.H_kv * p.B;
    return (Wh != W && n_wg > device_cus()) ? launch_decode_waves<D, Wh, kAppend, kRope>(p, stream)
                                            : launch_decode_waves<D, W, kAppend, kRope>(p, stream);
  }
}

// Partials buffer: part_m | part_l | part_acc (fp32), each region 256-byte aligned.
struct PartLayout {
  int64_t m, l, acc, total;
};

// rows: B * H_q * S for an unplanned launch, n_workgroups * G for a planned one
static PartLayout part_layout_rows(int64_t rows, int64_t D) {
  auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  PartLayout w;
  w.m = 0;
  w.l = up(rows * 4);
  w.acc = up(w.l + rows * 4);
  w.total = up(w.acc + rows * D * 4);
  return w;
}
static PartLayout part_layout(int64_t B, int64_t H_q, int64_t D, int64_t S) {
  return part_layout_rows(B * H_q * S, D);
}

// n_splits: the split count of an unplanned launch, or the workgroups of a
// planned one (p.plan set; lens / slot_ids / n_slots then unused).
template <bool kAppend, bool kRope, bool kPlanned = false>
static int decode_entry(DecodeParams& p, void* partials, int32_t* counters, int64_t B,
                        int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size, int64_t n_pages,
                        int64_t pool_page_stride, int64_t pool_head_stride, int64_t bt_stride,
                        int64_t bt_width, int64_t n_slots, int64_t n_splits, int32_t* err,
                        void* stream) {
  if (B < 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || n_pages <= 0 || bt_width <= 0 ||
      bt_stride < bt_width || (!kPlanned && n_slots <= 0) || n_splits <= 0 || page_size <= 0)
    return CIE_EINVAL;
  if (B == 0) return CIE_OK;
  if (!p.o || !p.q || !p.k_pool || !p.v_pool || !p.block_table) return CIE_EINVAL;
  if (kPlanned ? !p.plan : (!p.lens || !p.slot_ids)) return CIE_EINVAL;
  const int64_t G = H_q / H_kv;
  if constexpr (kPlanned) {
    // every (sequence, kv head) has at least one workgroup, at most kMaxSplits
    if (n_splits < B * H_kv || n_splits % H_kv != 0 || n_splits > B * H_kv * kMaxSplits)
      return CIE_EINVAL;
    if (n_splits > B * H_kv && (!partials || !counters)) return CIE_EINVAL;
  } else {
    if (n_splits > 1 && (!partials || !counters)) return CIE_EINVAL;
  }
  if (G > 16 || page_size % 16 != 0 || B > 65535 || H_kv > 65535 ||
      (!kPlanned && n_splits > kMaxSplits) || n_splits > 0x7fffffff ||
      bt_width * page_size > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  if (D != 64 && D != 128) return CIE_EUNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(p.o) | reinterpret_cast<uintptr_t>(p.q) |
       reinterpret_cast<uintptr_t>(p.k_pool) |
       reinterpret_cast<uintptr_t>(p.v_pool) | reinterpret_cast<uintptr_t>(partials) |
       reinterpret_cast<uintptr_t>(counters)) & 15)
    return CIE_EINVAL;
  if (pool_page_stride % 8 != 0 || pool_head_stride % 8 != 0) return CIE_EINVAL;

  const PartLayout w = kPlanned ? part_layout_rows(n_splits * G, D) : part_layout(B, H_q, D, n_splits);
  char* ws = static_cast<char*>(partials);
  p.part_m = reinterpret_cast<float*>(ws + w.m);
  p.part_l = reinterpret_cast<float*>(ws + w.l);
  p.part_acc = reinterpret_cast<float*>(ws + w.acc);
  p.counters = counters;
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
  p.n_splits = kPlanned ? 0 : (int32_t)n_splits;
  p.n_wg = kPlanned ? (int32_t)n_splits : 0;
  p.scale_log2 = kLog2e / __builtin_sqrtf((float)D);
  p.err = err;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_decode<64, kAppend, kRope, kPlanned>(p, s)
                 : launch_decode<128, kAppend, kRope, kPlanned>(p, s);
}

}  // namespace cie

using namespace cie;

extern "C" int64_t cie_paged_decode_partials_bytes(int64_t B, int64_t H_q, int64_t D,
                                                   int64_t n_splits) {
  if (B < 0 || H_q <= 0 || D <= 0 || n_splits <= 0) return -1;
  return part_layout(B, H_q, D, n_splits).total;
}

extern "C" int cie_paged_decode_max_splits(void) { return kMaxSplits; }

#ifdef CIE_DECODE_TRACE
// Trace builds only: where the decode kernels stamp their phases (device
// buffer of 24 uint64 per workgroup; NULL turns the stamps off).
extern "C" int cie_decode_trace_buffer(void* buf) {
  uint64_t* p = static_cast<uint64_t*>(buf);
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_decode_trace), &p, sizeof(p));
}
#endif

extern "C" int cie_paged_decode(void* o, const void* q, const void* k_pool, const void* v_pool,
                                const int64_t* lens, const int64_t* slot_ids,
                                const int64_t* block_table, void* partials, int32_t* counters,
                                int64_t B, int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size,
                                int64_t n_pages, int64_t pool_page_stride,
                                int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
                                int64_t n_slots, int64_t n_splits, int32_t* err, void* stream) {
  DecodeParams p{};
  p.o = static_cast<f16*>(o);
  p.q = static_cast<const f16*>(q);
  p.k_pool = const_cast<f16*>(static_cast<const f16*>(k_pool));
  p.v_pool = const_cast<f16*>(static_cast<const f16*>(v_pool));
  p.q_row_stride = H_q * D;
  p.lens = lens;
  p.slot_ids = slot_ids;
  p.block_table = block_table;
  return decode_entry<false, false>(p, partials, counters, B, H_q, H_kv, D, page_size, n_pages, pool_page_stride,
                             pool_head_stride, bt_stride, bt_width, n_slots, n_splits, err,
                             stream);
}

extern "C" int cie_paged_decode_append(
    void* o, const void* q, void* k_pool, void* v_pool, const void* k_new, const void* v_new,
    int64_t k_tok_stride, int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
    const int64_t* lens, const int64_t* slot_ids, const int64_t* block_table, void* partials,
    int32_t* counters, int64_t B, int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size, int64_t n_pages,
    int64_t pool_page_stride, int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
    int64_t n_slots, int64_t n_splits, int32_t* err, void* stream) {
  if (B > 0 && (!k_new || !v_new)) return CIE_EINVAL;
  if (((reinterpret_cast<uintptr_t>(k_new) | reinterpret_cast<uintptr_t>(v_new)) & 15) ||
      k_tok_stride % 8 != 0 || k_head_stride % 8 != 0 || v_tok_stride % 8 != 0 ||
      v_head_stride % 8 != 0)
    return CIE_EINVAL;
  DecodeParams p{};
  p.o = static_cast<f16*>(o);
  p.q = static_cast<const f16*>(q);
  p.k_pool = static_cast<f16*>(k_pool);
  p.v_pool = static_cast<f16*>(v_pool);
  p.k_new = static_cast<const f16*>(k_new);
  p.v_new = static_cast<const f16*>(v_new);
  p.k_tok_stride = k_tok_stride;
  p.k_head_stride = k_head_stride;
  p.v_tok_stride = v_tok_stride;
  p.v_head_stride = v_head_stride;
  p.q_row_stride = H_q * D;
  p.lens = lens;
  p.slot_ids = slot_ids;
  p.block_table = block_table;
  return decode_entry<true, false>(p, partials, counters, B, H_q, H_kv, D, page_size, n_pages,
                                   pool_page_stride, pool_head_stride, bt_stride, bt_width,
                                   n_slots, n_splits, err, stream);
}

extern "C" int cie_paged_decode_qkv_rope(
    void* o, const void* qkv, int64_t qkv_row_stride, const void* cos, const void* sin,
    int64_t cs_row_stride, void* k_pool, void* v_pool, const int64_t* lens,
    const int64_t* slot_ids, const int64_t* block_table, void* partials, int32_t* counters,
    int64_t B, int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size, int64_t n_pages,
    int64_t pool_page_stride, int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
    int64_t n_slots, int64_t n_splits, int32_t* err, void* stream) {
  if (B < 0 || H_q <= 0 || H_kv <= 0 || D <= 0) return CIE_EINVAL;
  if (B > 0 && (!qkv || !cos || !sin)) return CIE_EINVAL;
  if (((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(cos) |
        reinterpret_cast<uintptr_t>(sin)) & 15) ||
      qkv_row_stride % 8 != 0 || cs_row_stride % 8 != 0 ||
      qkv_row_stride < (H_q + 2 * H_kv) * D || cs_row_stride < D)
    return CIE_EINVAL;
  const f16* base = static_cast<const f16*>(qkv);
  DecodeParams p{};
  p.o = static_cast<f16*>(o);
  p.q = base;
  p.q_row_stride = qkv_row_stride;
  p.cos = static_cast<const f16*>(cos);
  p.sin = static_cast<const f16*>(sin);
  p.cs_stride = cs_row_stride;
  p.k_pool = static_cast<f16*>(k_pool);
  p.v_pool = static_cast<f16*>(v_pool);
  p.k_new = base + H_q * D;
  p.v_new = base + (H_q + H_kv) * D;
  p.k_tok_stride = qkv_row_stride;
  p.k_head_stride = D;
  p.v_tok_stride = qkv_row_stride;
  p.v_head_stride = D;
  p.lens = lens;
  p.slot_ids = slot_ids;
  p.block_table = block_table;
  return decode_entry<true, true>(p, partials, counters, B, H_q, H_kv, D, page_size, n_pages,
                                  pool_page_stride, pool_head_stride, bt_stride, bt_width,
                                  n_slots, n_splits, err, stream);
}

// ---------------------------------------------------------------------------
// Planned decode: cie_paged_decode_plan once per decode step, then one
// planned launch per layer.
extern "C" int64_t cie_paged_decode_plan_workgroups(int64_t B, int64_t H_kv, int64_t n_splits) {
  if (B <= 0 || H_kv <= 0 || n_splits < 0 || n_splits > kMaxSplits) return -1;
  if (n_splits > 0) return B * H_kv * n_splits;
  // the library's default: about one workgroup per CU (one resident round),
  // at least one and at most kMaxSplits per (sequence, kv head)
  int64_t per_head = (device_cus() + H_kv - 1) / H_kv;
  if (per_head < B) per_head = B;
  if (per_head > B * kMaxSplits) per_head = B * kMaxSplits;
  return H_kv * per_head;
}

extern "C" int64_t cie_paged_decode_plan_bytes(int64_t n_workgroups) {
  if (n_workgroups <= 0) return -1;
  return n_workgroups * (kPlanDescWords + kPlanWaves * kWave) * (int64_t)sizeof(int32_t);
}

extern "C" int64_t cie_paged_decode_planned_partials_bytes(int64_t n_workgroups, int64_t H_q,
                                                           int64_t H_kv, int64_t D) {
  if (n_workgroups <= 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || D <= 0) return -1;
  return part_layout_rows(n_workgroups * (H_q / H_kv), D).total;
}

extern "C" int cie_paged_decode_plan(void* plan, const int64_t* lens, const int64_t* slot_ids,
                                     const int64_t* block_table, int64_t B, int64_t H_kv,
                                     int64_t page_size, int64_t n_pages, int64_t bt_stride,
                                     int64_t bt_width, int64_t n_slots, int64_t append,
                                     int64_t n_workgroups, int32_t* err, void* stream) {
  if (B < 0 || H_kv <= 0 || page_size <= 0 || n_pages <= 0 || bt_width <= 0 ||
      bt_stride < bt_width || n_slots <= 0 || (append != 0 && append != 1))
    return CIE_EINVAL;
  if (B == 0) return CIE_OK;
  if (!plan || !lens || !slot_ids || !block_table) return CIE_EINVAL;
  if (n_workgroups < B * H_kv || n_workgroups % H_kv != 0 || n_workgroups > B * H_kv * kMaxSplits)
    return CIE_EINVAL;
  if (B > kPlanMaxSeqs || page_size % 16 != 0 || n_workgroups > 0x7fffffff ||
      bt_width * page_size > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(plan) & 15) return CIE_EINVAL;
  PlanParams q{};
  q.plan = static_cast<int32_t*>(plan);
  q.lens = lens;
  q.slot_ids = slot_ids;
  q.block_table = block_table;
  q.bt_stride = bt_stride;
  q.n_pages = n_pages;
  q.B = (int32_t)B;
  q.H_kv = (int32_t)H_kv;
  q.page_size = (int32_t)page_size;
  q.bt_width = (int32_t)bt_width;
  q.n_slots = (int32_t)(n_slots > 0x7fffffff ? 0x7fffffff : n_slots);
  q.n_wg = (int32_t)n_workgroups;
  q.append = (int32_t)append;
  q.err = err;
  hipLaunchKernelGGL(decode_plan_kernel, dim3((unsigned)n_workgroups), dim3(kPlanThreads), 0,
                     static_cast<hipStream_t>(stream), q);
  return (int)hipGetLastError();
}

extern "C" int cie_paged_decode_planned(void* o, const void* q, const void* k_pool,
                                        const void* v_pool, const int32_t* plan,
                                        const int64_t* block_table, void* partials,
                                        int32_t* counters, int64_t B, int64_t H_q, int64_t H_kv,
                                        int64_t D, int64_t page_size, int64_t n_pages,
                                        int64_t pool_page_stride, int64_t pool_head_stride,
                                        int64_t bt_stride, int64_t bt_width, int64_t n_workgroups,
                                        int32_t* err, void* stream) {
  DecodeParams p{};
  p.o = static_cast<f16*>(o);
  p.q = static_cast<const f16*>(q);
  p.k_pool = const_cast<f16*>(static_cast<const f16*>(k_pool));
  p.v_pool = const_cast<f16*>(static_cast<const f16*>(v_pool));
  p.q_row_stride = H_q * D;
  p.plan = plan;
  p.block_table = block_table;
  return decode_entry<false, false, true>(p, partials, counters, B, H_q, H_kv, D, page_size, n_pages,
                                          pool_page_stride, pool_head_stride, bt_stride, bt_width,
                                          0, n_workgroups, err, stream);
}

extern "C" int cie_paged_decode_append_planned(
    void* o, const void* q, void* k_pool, void* v_pool, const void* k_new, const void* v_new,
    int64_t k_tok_stride, int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
    const int32_t* plan, const int64_t* block_table, void* partials, int32_t* counters, int64_t B,
    int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size, int64_t n_pages,
    int64_t pool_page_stride, int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
    int64_t n_workgroups, int32_t* err, void* stream) {
  if (B > 0 && (!k_new || !v_new)) return CIE_EINVAL;
  if (((reinterpret_cast<uintptr_t>(k_new) | reinterpret_cast<uintptr_t>(v_new)) & 15) ||
      k_tok_stride % 8 != 0 || k_head_stride % 8 != 0 || v_tok_stride % 8 != 0 ||
      v_head_stride % 8 != 0)
    return CIE_EINVAL;
  DecodeParams p{};
  p.o = static_cast<f16*>(o);
  p.q = static_cast<const f16*>(q);
  p.k_pool = static_cast<f16*>(k_pool);
  p.v_pool = static_cast<f16*>(v_pool);
  p.k_new = static_cast<const f16*>(k_new);
  p.v_new = static_cast<const f16*>(v_new);
  p.k_tok_stride = k_tok_stride;
  p.k_head_stride = k_head_stride;
  p.v_tok_stride = v_tok_stride;
  p.v_head_stride = v_head_stride;
  p.q_row_stride = H_q * D;
  p.plan = plan;
  p.block_table = block_table;
  return decode_entry<true, false, true>(p, partials, counters, B, H_q, H_kv, D, page_size, n_pages,
                                         pool_page_stride, pool_head_stride, bt_stride, bt_width, 0,
                                         n_workgroups, err, stream);
}

extern "C" int cie_paged_decode_qkv_rope_planned(
    void* o, const void* qkv, int64_t qkv_row_stride, const void* cos, const void* sin,
    int64_t cs_row_stride, void* k_pool, void* v_pool, const int32_t* plan,
    const int64_t* block_table, void* partials, int32_t* counters, int64_t B, int64_t H_q,
    int64_t H_kv, int64_t D, int64_t page_size, int64_t n_pages, int64_t pool_page_stride,
    int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width, int64_t n_workgroups,
    int32_t* err, void* stream) {
  if (B < 0 || H_q <= 0 || H_kv <= 0 || D <= 0) return CIE_EINVAL;
  if (B > 0 && (!qkv || !cos || !sin)) return CIE_EINVAL;
  if (((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(cos) |
        reinterpret_cast<uintptr_t>(sin)) & 15) ||
      qkv_row_stride % 8 != 0 || cs_row_stride % 8 != 0 ||
      qkv_row_stride < (H_q + 2 * H_kv) * D || cs_row_stride < D)
    return CIE_EINVAL;
  const f16* base = static_cast<const f16*>(qkv);
  DecodeParams p{};
  p.o = static_cast<f16*>(o);
  p.q = base;
  p.q_row_stride = qkv_row_stride;
  p.cos = static_cast<const f16*>(cos);
  p.sin = static_cast<const f16*>(sin);
  p.cs_stride = cs_row_stride;
  p.k_pool = static_cast<f16*>(k_pool);
  p.v_pool = static_cast<f16*>(v_pool);
  p.k_new = base + H_q * D;
  p.v_new = base + (H_q + H_kv) * D;
  p.k_tok_stride = qkv_row_stride;
  p.k_head_stride = D;
  p.v_tok_stride = qkv_row_stride;
  p.v_head_stride = D;
  p.plan = plan;
  p.block_table = block_table;
  return decode_entry<true, true, true>(p, partials, counters, B, H_q, H_kv, D, page_size, n_pages,
                                        pool_page_stride, pool_head_stride, bt_stride, bt_width, 0,
                                        n_workgroups, err, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of cie_paged_decode_append: the split partials and
// arrival counters live in this file-scope device array instead of caller
// buffers.  Each GPU holds its own copy for the life of the process; host
// code reaches it only through the address hipGetSymbolAddress returns for
// the current device (the array's name is a host-side stand-in, not a device
// address).
namespace cie {

constexpr int64_t kScratchPartialBytes = int64_t(4) << 20;  // split partials
constexpr int64_t kScratchCounterWords = 16384;             // 2 * B * H_kv arrival + stale words
constexpr int64_t kScratchBytes = kScratchPartialBytes + kScratchCounterWords * 4;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void zero_words_kernel(int32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

struct ScratchSlot {
  char* ptr = nullptr;
  bool zeroed = false;
};

// The current device's scratch address; its counters are zeroed by a fill
// kernel on `stream` the first time (a kernel, not a memset, so a first call
// under graph capture records a kernel node).  Returns a CIE_* / hipError_t.
static int device_scratch(hipStream_t stream, char** out) {
  constexpr int kMaxDevices = 64;
  static ScratchSlot slots[kMaxDevices];
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return CIE_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(mu);
  ScratchSlot& s = slots[dev];
  if (s.ptr == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    s.ptr = static_cast<char*>(ptr);
  }
  if (!s.zeroed) {
    hipLaunchKernelGGL(zero_words_kernel, dim3(16), dim3(256), 0, stream,
                       reinterpret_cast<int32_t*>(s.ptr + kScratchPartialBytes), kScratchCounterWords);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    s.zeroed = true;
  }
  *out = s.ptr;
  return CIE_OK;
}

}  // namespace cie

// Whether a problem fits the static scratch: the partials (none for one split)
// and, past one split, 2 * B * H_kv counter words.
static bool noalloc_fits(int64_t B, int64_t H_q, int64_t H_kv, int64_t D, int64_t n_splits) {
  if (n_splits == 1) return true;
  return 2 * B * H_kv <= kScratchCounterWords &&
         part_layout(B, H_q, D, n_splits).total <= kScratchPartialBytes;
}

extern "C" int64_t cie_paged_decode_noalloc_limit(int64_t H_q, int64_t H_kv, int64_t D,
                                                  int64_t n_splits) {
  // largest batch the entry point accepts: scratch, and the kernel's grid limit
  if (H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || D <= 0 || n_splits <= 0 ||
      n_splits > kMaxSplits)
    return -1;
  constexpr int64_t kMaxBatch = 65535;
  int64_t lo = 0, hi = kMaxBatch;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (noalloc_fits(mid, H_q, H_kv, D, n_splits))
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

extern "C" int cie_paged_decode_append_noalloc(
    void* o, const void* q, void* k_pool, void* v_pool, const void* k_new, const void* v_new,
    int64_t k_tok_stride, int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
    const int64_t* lens, const int64_t* slot_ids, const int64_t* block_table, int64_t B,
    int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size, int64_t n_pages,
    int64_t pool_page_stride, int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
    int64_t n_slots, int64_t n_splits, int32_t* err, void* stream) {
  if (B < 0 || H_q <= 0 || H_kv <= 0 || D <= 0 || n_splits <= 0) return CIE_EINVAL;
  if (B == 0) return CIE_OK;
  if (n_splits > kMaxSplits || B > 65535) return CIE_EUNSUPPORTED;
  if (!noalloc_fits(B, H_q, H_kv, D, n_splits)) return CIE_ESCRATCH;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = nullptr;
  const int rc = device_scratch(s, &ws);
  if (rc != CIE_OK) return rc;
  return cie_paged_decode_append(o, q, k_pool, v_pool, k_new, v_new, k_tok_stride, k_head_stride,
                                 v_tok_stride, v_head_stride, lens, slot_ids, block_table, ws,
                                 reinterpret_cast<int32_t*>(ws + kScratchPartialBytes), B, H_q,
                                 H_kv, D, page_size, n_pages, pool_page_stride, pool_head_stride,
                                 bt_stride, bt_width, n_slots, n_splits, err, stream);
}
