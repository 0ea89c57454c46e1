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
// row of the tile inside the MFMA.  One work item is (tile, column group,
// key chunk): a column group is up to col_group<D>() column tiles (half as
// many for a sequence whose tiles all have short key ranges: seq_cg), and a
// tile's key range [0, kv_len + last row + 1) is cut into chunks only when it
// is longer than kWavePairs 32-key steps per wave (CIE_MIXED_NARROW_PAIRS for
// a tile of one column tile, e.g. a decode row).  The item's key tiles are
// split over the workgroup's waves; every wave carries all of the group's
// column tiles, so each K/V byte is loaded once per workgroup and reused by
// every column of the group in registers.  The waves fold their states
// through LDS in one round (wave c combines column tile c).  A single-chunk
// item writes o directly.  Otherwise each chunk writes its partial (m, l, acc) per column
// with device-coherent stores and the last chunk to arrive (counter per
// tile and column group) merges them with log-sum-exp, writes o and resets
// the counter.  Partials are packed per launch: only split tiles have rows,
// sequence by sequence, within a budget the caller's buffer sets; a
// sequence past it runs unsplit (see the tile runs below).  Every workgroup
// plans the batch (item counts, dealing order, partial bases) at its start;
// a planned launch reads that plan, made once per mixed step by
// mixed_plan_kernel, instead.  The reference instead walks a tile's whole
// prefix with one program and pads every L = 1 sequence to a 16-row tile
// (prefill_attention.py:49-50, 93).
#include "attn_engine.h"

namespace cie {

// Build-time tuning (defaults are the shipped configuration):
//   CIE_MIXED_WAVES        wavefronts per workgroup (D = 64)
//   CIE_MIXED_CG           column tiles per work item (D = 64)
//   CIE_MIXED_WAVE_PAIRS   32-key steps per wave before a tile's keys are
//                          split over several workgroups
//   CIE_MIXED_NARROW_PAIRS the same for a tile of one column tile (a decode
//                          row: its steps are cheap, its keys many, so it is
//                          split sooner and its chunks spread over idle
//                          workgroups; 12 measured faster than 8, 16 or 32
//                          at config 3: a chunk's fixed cost, not its few
//                          steps, sets its time)
//   CIE_MIXED_PF           32-key steps of loads in flight per wave (D = 64)
//   CIE_MIXED_QLDS         1: the item's Q operands live in LDS (one copy per
//                          workgroup), not registers (a wave then fits 256
//                          registers at D = 64)
//   CIE_MIXED_WG_PER_CU    workgroups per CU in the grid
//   CIE_MIXED_SHORT_KTILES a sequence whose longest tile has at most this
//                          many 16-key tiles uses column groups of half
//                          CIE_MIXED_CG (0: never)
//   CIE_MIXED_LONG_KTILES  the same for a sequence whose longest tile has at
//                          least this many (0: never; 96 and 128 measured
//                          slower at config 3: 24.6 against 21.7 us)
#ifndef CIE_MIXED_WAVES
#define CIE_MIXED_WAVES 4
#endif
#ifndef CIE_MIXED_CG
#define CIE_MIXED_CG 4
#endif
#ifndef CIE_MIXED_WAVE_PAIRS
#define CIE_MIXED_WAVE_PAIRS 24
#endif
#ifndef CIE_MIXED_PF
#define CIE_MIXED_PF 1
#endif
#ifndef CIE_MIXED_QLDS
#define CIE_MIXED_QLDS 1
#endif
#ifndef CIE_MIXED_WG_PER_CU
#define CIE_MIXED_WG_PER_CU 1
#endif
#ifndef CIE_MIXED_PIPELINED
#define CIE_MIXED_PIPELINED 1
#endif
#ifndef CIE_MIXED_NARROW_PAIRS
#define CIE_MIXED_NARROW_PAIRS 12
#endif
#ifndef CIE_MIXED_NARROW_PF
#define CIE_MIXED_NARROW_PF 1
#endif
#ifndef CIE_MIXED_NARROW_NT
#define CIE_MIXED_NARROW_NT 1
#endif
#ifndef CIE_MIXED_NARROW_ORDER
#define CIE_MIXED_NARROW_ORDER 0
#endif
#ifndef CIE_MIXED_SHORT_KTILES
#define CIE_MIXED_SHORT_KTILES 32
#endif
#ifndef CIE_MIXED_LONG_KTILES
#define CIE_MIXED_LONG_KTILES 0
#endif

constexpr int kWavePairs = CIE_MIXED_WAVE_PAIRS;
constexpr int kMaxChunks = 16;    // workgroups per (tile, column group) at most
constexpr int kMaxColGroups = 8;  // column groups per tile at most (<= 8 column tiles)
// Partial rows a launch uses at most, whatever the buffer: with each
// sequence's rows clamped to the budget + 1, the plan's prefix over kMaxSeqs
// sequences stays below 2^31.
constexpr int64_t kMaxPartRows = (1 << 21) - 64;


// Wavefronts per workgroup, column tiles per work item (registers: 16*NT
// accumulators each) and load prefetch depth (registers: one 32-key K/V step
// each).  D = 128 runs 4 waves (one per SIMD, so each may use 512 registers).
template <int D>
constexpr int mixed_waves() {
  return D <= 64 ? CIE_MIXED_WAVES : 4;
}
template <int D>
constexpr int col_group() {
  return D <= 64 ? CIE_MIXED_CG : 1;
}
// The key stream of a work item when the pools are under 4 GiB: of several
// column tiles at D = 64, stream_tiles_pipelined (steps overlapped, one
// descriptor per pool); else stream_tiles_pool (one descriptor per pool).
// Pools of 4 GiB or more: stream_tiles (a descriptor per tile).
template <int D>
constexpr bool mixed_pipelined() {
  return D == 64 && CIE_MIXED_PIPELINED;
}
template <int D>
constexpr int mixed_pf() {
  return D <= 64 ? CIE_MIXED_PF : 1;
}
// The same for a work item of one column tile (a decode row): its steps are
// short, so more of them are kept in flight.
template <int D, int NCT>
constexpr int stream_pf() {
  return D <= 64 && NCT == 1 ? CIE_MIXED_NARROW_PF : mixed_pf<D>();
}

// LDS slot of wave w's state of column tile c in the fold (wave c folds
// column tile c and keeps its own state in registers: W - 1 slots a tile).
template <int W>
__device__ __forceinline__ int fold_slot(int w, int c) {
  return c * (W - 1) + (w < c ? w : w - 1);
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
  float* part_m;    // [part_cap] split-chunk partial rows (m): packed, see the tile runs
  float* part_l;    // [part_cap]
  float* part_acc;  // [part_cap][D]
  int64_t part_cap;  // partial rows the caller's buffer holds (<= kMaxPartRows)
  int32_t* counters;  // 2 x [B][H_kv][n_qtiles][kMaxColGroups]: arrival words, then stale words
  int64_t pool_page_stride, pool_head_stride, bt_stride, n_pages, total_T;
  int32_t bt_width, n_slots, B, H_q, H_kv, G, page_size, n_qtiles;
  uint32_t g_magic, tpp_magic;  // div_magic(G), div_magic(page_size / 16)
  uint32_t pool_bytes;          // bytes of each pool if under 4 GiB, else 0
  float scale_log2;
  int32_t* err;
  // planned launches: the step's plan (cie_mixed_plan) and its capacity in
  // items; the plan kernel writes `plan_out`
  const int32_t* plan;
  int32_t* plan_out;
  int32_t plan_cap;
};

struct SeqInfo {
  int64_t t0;  // first packed row
  int64_t slot;
  int L;  // query rows
  int c;  // prior kv length
  // first partial row of the sequence's split tiles, or -1: its tiles are
  // not split (the batch's partial rows would exceed the caller's buffer)
  int pbase;
};

__device__ __forceinline__ SeqInfo seq_info(const MixedParams& p, int b) {
  SeqInfo s{0, 0, 0, 0, 0};
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
  int row0, rows, n_combos, n_ctiles, cg, n_groups, key_end, n_ktiles, n_pairs, n_chunks;
  int pblk;  // first partial row of a split tile's block (set per work item: part_region)
};

// Column tiles per group for every tile of a sequence: CG, or CG / 2 when
// the sequence's last (longest) tile has at most CIE_MIXED_SHORT_KTILES key
// tiles.  Such items are short, so a launch of them is set by latency, and
// splitting their columns over twice the workgroups shortens it more than
// the extra K/V reads cost; long tiles keep every K/V byte shared by CG
// column tiles.  A function of the sequence alone, so the plan, the item
// lookup and the item agree.
template <int CG>
__device__ __forceinline__ int seq_cg(const SeqInfo& s) {
  if constexpr (CG < 4) return CG;
  const int kt = (s.c + s.L + 15) >> 4;
  if (CIE_MIXED_SHORT_KTILES > 0 && kt <= CIE_MIXED_SHORT_KTILES) return CG / 2;
  if (CIE_MIXED_LONG_KTILES > 0 && kt >= CIE_MIXED_LONG_KTILES) return CG / 2;
  return CG;
}

// Column groups of n column tiles at cg per group (cg = CG or CG / 2: both
// divisions by constants).
template <int CG>
__device__ __forceinline__ int n_col_groups(int n, int cg) {
  if constexpr (CG < 2)
    return n;
  else
    return cg == CG ? (n + CG - 1) / CG : (n + CG / 2 - 1) / (CG / 2);
}

// CG = column tiles per group, W = wavefronts per workgroup (template
// arguments, so the chunk count divides by constants: a work item's lookup
// walks its sequence's tiles, and a run-time division per tile cost ~2 us on
// the last tiles of a 2,304-key sequence).
template <int CG, int W>
__device__ __forceinline__ TilePlan tile_plan(int qt, const SeqInfo& s, int G) {
  TilePlan t;
  t.row0 = qt * 16;
  t.rows = min(16, s.L - t.row0);
  t.n_combos = t.rows * G;
  t.n_ctiles = (t.n_combos + 15) >> 4;
  t.cg = seq_cg<CG>(s);
  t.n_groups = n_col_groups<CG>(t.n_ctiles, t.cg);
  t.key_end = s.c + t.row0 + t.rows;
  t.n_ktiles = (t.key_end + 15) >> 4;
  t.n_pairs = (t.n_ktiles + 1) >> 1;
  constexpr int kPerNarrow = W * CIE_MIXED_NARROW_PAIRS;
  constexpr int kPerWide = W * kWavePairs;
  const int chunks = t.n_ctiles == 1 ? (t.n_pairs + kPerNarrow - 1) / kPerNarrow
                                     : (t.n_pairs + kPerWide - 1) / kPerWide;
  t.n_chunks = s.pbase < 0 ? 1 : max(1, min(kMaxChunks, chunks));
  t.pblk = 0;
  return t;
}

// Key tiles [*t0, *t1) of part i of n when a tile's 32-key steps are split
// into n near-equal runs (run boundaries on whole steps).
// (32-bit arithmetic: a tile has fewer than 2^27 key tiles — the launch
// rejects block tables of 2^31 keys — and i < n <= kMaxChunks, so
// steps * (i + 1) < 2^31)
__device__ __forceinline__ void split_steps(int t_begin, int t_end, int i, int n, int& t0, int& t1) {
  const uint32_t steps = (uint32_t)(t_end - t_begin + 1) >> 1;
  t0 = min(t_end, t_begin + 2 * (int)(steps * (uint32_t)i / (uint32_t)n));
  t1 = min(t_end, t_begin + 2 * (int)(steps * (uint32_t)(i + 1) / (uint32_t)n));
}

// As split_steps, with the remainder steps on the first parts: a tile's last
// part holds its diagonal (masked) step, so the wave that takes it is not
// also the one given an extra step.
__device__ __forceinline__ void split_steps_front(int t_begin, int t_end, int i, int n, int& t0,
                                                  int& t1) {
  const uint32_t steps = (uint32_t)(t_end - t_begin + 1) >> 1;
  const uint32_t un = (uint32_t)n;
  t0 = min(t_end, t_begin + 2 * (int)((steps * (uint32_t)i + un - 1) / un));
  t1 = min(t_end, t_begin + 2 * (int)((steps * (uint32_t)(i + 1) + un - 1) / un));
}

// Q^T operand and key limit of column tile ct (columns = (row, head) pairs).
template <int D>
__device__ __forceinline__ void load_combo_q(const MixedParams& p, const SeqInfo& s,
                                             const TilePlan& tp, int g, int ct, int r16, int grp,
                                             f16x8 (&qop)[Geo<D>::KS], int& lim) {
  const int cc = ct * 16 + r16;
  if (cc < tp.n_combos) {
    const int row = magic_div(cc, p.g_magic);
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

// Key limit of column tile ct's lane column (load_combo_q's lim alone).
__device__ __forceinline__ int combo_lim(const MixedParams& p, const SeqInfo& s,
                                         const TilePlan& tp, int ct, int r16) {
  const int cc = ct * 16 + r16;
  return cc < tp.n_combos ? s.c + tp.row0 + magic_div(cc, p.g_magic) + 1 : tp.key_end;
}

// Row of column cc of the tile relative to the tile's first row's first q
// head, in units of (row, q head) = H_q * (row) + g * G + head - ...; i.e. the
// index into [(t0 + row0) * H_q, ...) of the tile's partial / output rows.
__device__ __forceinline__ int column_off(const MixedParams& p, int g, int cc) {
  const int row = magic_div(cc, p.g_magic);
  const int head = cc - row * p.G;
  return row * p.H_q + g * p.G + head;
}

// Profiling builds only (-DCIE_MIXED_TRACE): thread 0 stamps each work item's
// phases (s_memrealtime, 100 MHz) into LDS — LDS writes do not count in
// vmcnt, so the stamps add no wait on the K/V loads — and copies the item's
// 16 words to the buffer named by cie_mixed_trace_buffer() (exported by such
// builds alone) when the item ends, at [kv head][item][16].
#ifdef CIE_MIXED_TRACE
__device__ uint64_t* g_mixed_trace;
__shared__ uint64_t sm_mixed_trace[16];
#define MIXED_TRACE(item, k, v)                      \
  do {                                               \
    if (threadIdx.x == 0) sm_mixed_trace[(k)] = (v); \
  } while (0)
// every wave's first lane (slots 10 + wave: the waves' key-loop ends)
#define MIXED_TRACE_WAVE(k, v)                                                         \
  do {                                                                                 \
    if ((threadIdx.x & (kWave - 1)) == 0) sm_mixed_trace[(k) + threadIdx.x / kWave] = (v); \
  } while (0)
#define MIXED_TRACE_FLUSH(head, item)                                                   \
  do {                                                                                  \
    if (threadIdx.x == 0 && g_mixed_trace != nullptr && (item) < 4096) {                \
      for (int k_ = 0; k_ < 16; ++k_)                                                   \
        g_mixed_trace[((int64_t)(head) * 4096 + (item)) * 16 + k_] = sm_mixed_trace[k_]; \
      for (int k_ = 0; k_ < 16; ++k_)                                                   \
        if (k_ != 6 && k_ != 14 && k_ != 15) sm_mixed_trace[k_] = 0;                   \
    }                                                                                   \
  } while (0)
#else
#define MIXED_TRACE(item, k, v) \
  do {                          \
  } while (0)
#define MIXED_TRACE_WAVE(k, v) \
  do {                         \
  } while (0)
#define MIXED_TRACE_FLUSH(head, item) \
  do {                                \
  } while (0)
#endif

// Where a split tile's partial state lives: row column_off * n_chunks +
// chunk of the tile's block, which starts at row tp.pblk (the layout is
// described with the tile runs below).
struct PartRegion {
  __amdgpu_buffer_rsrc_t acc;  // over the tile's rows * H_q * n_chunks * D floats
  float* m;                    // the tile block's row 0 of part_m
  float* l;
};

template <int D>
__device__ __forceinline__ PartRegion part_region(const MixedParams& p, const TilePlan& tp) {
  PartRegion r;
  r.acc = coherent_rsrc(p.part_acc + (int64_t)tp.pblk * D,
                        (uint32_t)(tp.rows * p.H_q * tp.n_chunks * D * sizeof(float)));
  r.m = p.part_m + tp.pblk;
  r.l = p.part_l + tp.pblk;
  return r;
}

// One work item's waves: key tiles [w0, w1) against column tiles
// [ct0, ct0 + NCT); then the workgroup folds each column tile through LDS
// and writes o (single chunk) or the chunk's partial state.
template <int D, bool P32, int NCT>
__device__ __forceinline__ void run_group(const MixedParams& p, const SeqInfo& s,
                                          const TilePlan& tp, int g, int ct0, int chunk, int w0,
                                          int w1, const PagedSrc& src, int wave, int r16, int grp,
                                          f32x4* sm_facc, float2* sm_fml, f16x8* sm_q, int item) {
  constexpr int NT = Geo<D>::NT;
  constexpr int KS = Geo<D>::KS;
  constexpr int W = mixed_waves<D>();
  SoftmaxAcc<D, NCT> st;
  st.init();
  if constexpr (CIE_MIXED_QLDS) {
    // One copy of the item's Q operands per workgroup, in LDS: wave c loads
    // column tile c (every wave streams keys against all of them), and the
    // copy is written while each wave's first page ids are in flight, so the
    // Q loads and the page-id loads share one memory round trip; a barrier
    // then publishes it to every wave before the first step.
    static_assert(col_group<D>() <= W, "one wave per column tile of a group");
    int lim[NCT];
    f16x8 qw[KS];
    int lim_w;
#pragma unroll
    for (int c = 0; c < NCT; ++c) lim[c] = combo_lim(p, s, tp, ct0 + c, r16);
    const bool loads = wave < NCT;
    if (loads) load_combo_q<D>(p, s, tp, g, ct0 + wave, r16, grp, qw, lim_w);
    const int lane = opaque((int)threadIdx.x) & (kWave - 1);
    auto stage_q = [&]() {
      if (loads) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) sm_q[(wave * KS + ks) * kWave + lane] = qw[ks];
      }
      __syncthreads();
      MIXED_TRACE(item, 9, __builtin_amdgcn_s_memrealtime());
    };
    // the lane's column limits, as row offsets (< 16) packed a byte per
    // column tile over one base: a register, not NCT (read only on the
    // masked steps)
    uint32_t rows = 0;
#pragma unroll
    for (int c = 0; c < NCT; ++c) rows |= (uint32_t)(lim[c] - (s.c + tp.row0 + 1)) << (8 * c);
    const int lim_base = uniform(s.c + tp.row0 + 1);
    auto lims = [&](int c) { return lim_base + (int)((rows >> (8 * c)) & 0xffu); };
    if constexpr (P32 && mixed_pipelined<D>() && NCT >= 2)
      stream_tiles_pipelined<D, NCT>(st, QLds<D>{sm_q, lane}, lims, w0, w1, tp.key_end, src,
                                     p.scale_log2, r16, grp, stage_q);
    else if constexpr (P32)
      stream_tiles_pool<D, NCT, stream_pf<D, NCT>(), QLds<D>, decltype(stage_q),
                        NCT == 1 && CIE_MIXED_NARROW_NT ? kBufNt : 0>(
          st, QLds<D>{sm_q, lane}, lim, w0, w1, tp.key_end, src, p.scale_log2, r16, grp, stage_q);
    else
      stream_tiles<D, NCT, stream_pf<D, NCT>(), QLds<D>, decltype(stage_q),
                   NCT == 1 && CIE_MIXED_NARROW_NT ? kBufNt : 0>(
          st, QLds<D>{sm_q, lane}, lim, w0, w1, tp.key_end, src, p.scale_log2, r16, grp, stage_q);
  } else {
    f16x8 qop[NCT][KS];
    int lim[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c) load_combo_q<D>(p, s, tp, g, ct0 + c, r16, grp, qop[c], lim[c]);
    MIXED_TRACE(item, 9, __builtin_amdgcn_s_memrealtime());
    stream_tiles<D, NCT, mixed_pf<D>()>(st, QRegs<D, NCT>{qop}, lim, w0, w1, tp.key_end, src,
                                        p.scale_log2, r16, grp, [] {});
  }
  MIXED_TRACE(item, 8, __builtin_amdgcn_s_memrealtime());
  MIXED_TRACE_WAVE(10, __builtin_amdgcn_s_memrealtime());
  // Fold the waves' states in one round: every wave puts its states of the
  // other waves' column tiles into LDS in its register layout (one slot per
  // (wave, column tile), fold_slot), and after one barrier wave c combines
  // column tile c lane by lane — each lane reads its own (column, dims) slots
  // of the other waves' states, so the reads are conflict-free and the SIMDs
  // fold their tiles at once — and writes o (single chunk) or the chunk's
  // partial.  Nothing waits for the fold to end: the next item's first LDS
  // writes (its Q) touch no slot, and its own fold follows its Q barrier.
  static_assert(NCT <= W, "a wave per column tile of the group");
  // lane ids derived afresh: nothing lane-dependent of the fold is held in
  // registers through the key loop
  const int lane = opaque((int)threadIdx.x) & (kWave - 1);
  r16 = lane & 15;
  grp = lane >> 4;
  const int64_t tile_row0 = (s.t0 + tp.row0) * p.H_q;
  const PartRegion pr = part_region<D>(p, tp);  // (used only if tp.n_chunks > 1)
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    if (c == wave) continue;  // wave c keeps its own state in registers
    const int slot = fold_slot<W>(wave, c);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) sm_facc[(slot * NT + nt) * kWave + lane] = st.acc[c][nt];
    sm_fml[slot * kWave + lane] = float2{st.m[c], st.l(c)};
  }
  __syncthreads();
  {
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      if (c != wave) continue;
      float mw[W], lw[W];
#pragma unroll
      for (int w = 0; w < W; ++w) {
        if (w == c) {
          mw[w] = st.m[c];
          lw[w] = st.l(c);
        } else {
          const float2 ml = sm_fml[fold_slot<W>(w, c) * kWave + lane];
          mw[w] = ml.x;
          lw[w] = ml.y;
        }
      }
      float M = mw[0];
#pragma unroll
      for (int w = 1; w < W; ++w) M = fmaxf(M, mw[w]);
      // a state that saw no key holds kEmptyMax and weighs 2^(kEmptyMax - M)
      // = 0 (if every state is empty, M = kEmptyMax: den = 0 and o = 0)
      f32x4 num[NT];
      float den = 0.f;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) num[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float a = fast_exp2(mw[w] - M);
        den = __builtin_fmaf(a, lw[w], den);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          num[nt] += a * (w == c ? st.acc[c][nt]
                                 : sm_facc[(fold_slot<W>(w, c) * NT + nt) * kWave + lane]);
      }
      const int n_cols = min(16, tp.n_combos - (ct0 + c) * 16);
      if (r16 < n_cols) {
        // lane (r16, grp) holds dims NT * (4 * grp + r) + nt: 4 * NT
        // contiguous dims from 4 * NT * grp of column r16
        const int off = column_off(p, g, (ct0 + c) * 16 + r16);
        const int d0 = 4 * NT * grp;
        if (tp.n_chunks == 1) {
          const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
          for (int h = 0; h < NT / 2; ++h) {  // 8 dims per 16-byte store
            f16x8 v;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int k = 8 * h + e;  // dim d0 + k = d0 + NT * r + nt
              v[e] = (f16)(num[k % NT][k / NT] * inv);
            }
            *reinterpret_cast<f16x8*>(p.o + (tile_row0 + off) * D + d0 + 8 * h) = v;
          }
        } else {
          const int prow = off * tp.n_chunks + chunk;
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int nq = 0; nq < NT / 4; ++nq)
              agent_store4(pr.acc, (uint32_t)((prow * D + d0 + NT * r + 4 * nq) * sizeof(float)),
                           f32x4{num[4 * nq][r], num[4 * nq + 1][r], num[4 * nq + 2][r],
                                 num[4 * nq + 3][r]});
          if (grp == 0) {
            agent_store(pr.m + prow, M);
            agent_store(pr.l + prow, den);
          }
        }
      }
    }
  }
}

// Last chunk of a (tile, column group): combine the n_chunks partials of the
// group's columns into o.  A unit is 4 consecutive dims of one column
// (consecutive threads: consecutive dims, so every load is a whole-line
// 16-byte access); a thread holds up to kUnits units and, per group of four
// chunks, issues the loads of all of them before combining any, so a merge
// of up to four chunks is one memory round trip; chunks are combined with a
// running log-sum-exp.
template <int D>
__device__ __forceinline__ void merge_group(const MixedParams& p, const SeqInfo& s,
                                            const TilePlan& tp, int g, int ct0, int n_cols) {
  constexpr int kGroup = 4;
  constexpr int NTH = mixed_waves<D>() * kWave;
  constexpr int kUnits = (16 * col_group<D>() * (D / 4) + NTH - 1) / NTH;
  const int K = tp.n_chunks;
  const int n_units = n_cols * (D / 4);
  const int64_t tile_row0 = (s.t0 + tp.row0) * p.H_q;
  const PartRegion pr = part_region<D>(p, tp);
  const int tid = opaque((int)threadIdx.x);
  int off[kUnits], d4[kUnits];
  bool live[kUnits];
  float M[kUnits], den[kUnits];
  f32x4 num[kUnits];
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    const int it = tid + u * NTH;
    live[u] = it < n_units;
    const int j = live[u] ? it / (D / 4) : 0;
    d4[u] = (it - j * (D / 4)) * 4;
    off[u] = column_off(p, g, ct0 * 16 + j);
    M[u] = kNegInf;
    den[u] = 0.f;
    num[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int k0 = 0; k0 < K; k0 += kGroup) {
    float mk[kUnits][kGroup], lk[kUnits][kGroup];
    f32x4 val[kUnits][kGroup];
#pragma unroll
    for (int u = 0; u < kUnits; ++u)
#pragma unroll
      for (int c = 0; c < kGroup; ++c) {
        const int prow = off[u] * K + k0 + c;
        if (live[u] && k0 + c < K) {
          mk[u][c] = agent_load(pr.m + prow);
          lk[u][c] = agent_load(pr.l + prow);
          val[u][c] = agent_load4(pr.acc, (uint32_t)((prow * D + d4[u]) * sizeof(float)));
        } else {
          mk[u][c] = kNegInf;
          lk[u][c] = 0.f;
          val[u][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      float Mg = M[u];
#pragma unroll
      for (int c = 0; c < kGroup; ++c) Mg = fmaxf(Mg, mk[u][c]);
      if (Mg == kNegInf) continue;  // nothing attended so far
      const float rs = fast_exp2(M[u] - Mg);  // 0 when M = -inf
      den[u] *= rs;
      num[u] *= rs;
#pragma unroll
      for (int c = 0; c < kGroup; ++c) {
        const float a = mk[u][c] == kNegInf ? 0.f : fast_exp2(mk[u][c] - Mg);
        den[u] = __builtin_fmaf(a, lk[u][c], den[u]);
        num[u] += a * val[u][c];
      }
      M[u] = Mg;
    }
  }
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    if (!live[u]) continue;
    const float inv = den[u] > 0.f ? 1.f / den[u] : 0.f;
    const f16x4 h = {(f16)(num[u][0] * inv), (f16)(num[u][1] * inv), (f16)(num[u][2] * inv),
                     (f16)(num[u][3] * inv)};
    *reinterpret_cast<f16x4*>(p.o + (tile_row0 + off[u]) * D + d4[u]) = h;
  }
}

constexpr int kMaxSeqs = 1024;  // sequences a launch can plan (LDS plan tables)
// A step's plan (cie_mixed_plan): kPlanHeader header words, then 8 words per
// item; a planned launch stages the descriptors of its first kDescRounds
// rounds in LDS.
constexpr int kPlanHeader = 8;
constexpr int kDescRounds = 16;
constexpr int kRankSeqs = 64;   // batches up to this size deal their items heaviest first
static_assert(kRankSeqs == kWave, "a batch small enough to rank is planned by one wave");

// Bytes of the kernel's dynamic LDS: the plan tables of B sequences — t0
// and the partial base as an int2 (one read); slot, rows, prior, the order
// and the item prefix (B + 1 entries) as int32.  (t0 < total_T < 2^31: the
// launch bounds total_T * kMaxColGroups * kMaxChunks by 2^31.)
constexpr size_t mixed_plan_lds(int B) {
  return (size_t)B * sizeof(int2) + (size_t)(4 * B + (B + 1)) * sizeof(int);
}

// LDS one workgroup may allocate on gfx950.
constexpr size_t kLdsPerWorkgroup = 160 * 1024;

// A sequence's tiles and their items.  Full (16-row) tiles all have the same
// column groups and a chunk count that grows with the tile index: with
// c16 = ceil(prior / 16), full tile t has c16 + t + 1 key tiles and
// clamp(ceil((c16 + t + 1) / Q), 1, kMaxChunks) chunks for Q key tiles per
// chunk (tile_plan's rule), so the tiles group into runs of equal chunk
// count that are counted and searched without walking the tiles.  A
// sequence's items are walked heaviest first: its partial last tile (if
// any), then its full tiles from the top down.
struct SeqTiles {
  int n_tiles;  // query tiles computed (the grid's max_seqlen cap applied)
  int n_full;   // full tiles among them
  int c16;
  bool partial;  // tile n_tiles - 1 has fewer than 16 rows
  int ng_full;   // column groups of a full tile
  bool full_narrow;  // a full tile is one column tile (G = 1): narrow chunks
  bool split;        // the sequence has partial rows (pbase >= 0): tiles may chunk
};

template <int CG, int W>
__device__ __forceinline__ SeqTiles seq_tiles(const SeqInfo& s, int n_qtiles, int G) {
  SeqTiles t;
  t.n_tiles = min((s.L + 15) >> 4, n_qtiles);
  t.n_full = min(s.L >> 4, t.n_tiles);
  t.c16 = (s.c + 15) >> 4;
  t.partial = t.n_tiles > t.n_full;
  t.ng_full = n_col_groups<CG>(G, seq_cg<CG>(s));
  t.full_narrow = G <= 1;
  t.split = s.pbase >= 0;
  return t;
}

// Visit the runs of full tiles [0, n) with equal chunk counts (Q key tiles a
// chunk), from the top tile down: f(t_lo, t_hi, k) returns true to stop.
// (A sequence that may not split has one run, of one chunk: full_runs.)
template <int Q, class F>
__device__ __forceinline__ void chunk_runs(int n, int c16, F f) {
  for (int t_hi = n - 1; t_hi >= 0;) {
    const int k = min(kMaxChunks, (c16 + t_hi + 1 + Q - 1) / Q);
    // lowest tile with the same (clamped) count: c16 + t + 1 > (k - 1) * Q
    const int t_lo = k == 1 ? 0 : max(0, (k - 1) * Q - c16);
    if (f(t_lo, t_hi, k)) return;
    t_hi = t_lo - 1;
  }
}

template <int W>
constexpr int wide_chunk_ktiles() {
  return 2 * W * kWavePairs;
}
template <int W>
constexpr int narrow_chunk_ktiles() {
  return 2 * W * CIE_MIXED_NARROW_PAIRS;
}

template <int W, class F>
__device__ __forceinline__ void full_runs(const SeqTiles& st, F f) {
  if (!st.split) {
    if (st.n_full > 0) f(0, st.n_full - 1, 1);
  } else if (st.full_narrow) chunk_runs<narrow_chunk_ktiles<W>()>(st.n_full, st.c16, f);
  else chunk_runs<wide_chunk_ktiles<W>()>(st.n_full, st.c16, f);
}

// The partials of a launch are packed: only split tiles (two chunks or more)
// have any.  Sequence b's split tiles own rows [pbase_b, pbase_b + P_b) of
// the partial arrays — its full tiles in tile order, then its partial last
// tile — and tile t's block holds rows_t * H_q * chunks_t rows: row
// column_off * chunks_t + chunk, column_off = row * H_q + g * G + head (every
// kv head's columns).  pbase_b is the prefix of P_b over the batch in
// sequence order; a sequence whose block would end past the caller's buffer
// is not split at all (pbase = -1: one chunk per tile, no partials), so a
// launch never needs more than the buffer it was given, and parity does not
// depend on the budget (an unsplit tile is the same attention, later).

// First row of query tile qt's block within its sequence's partial rows.
template <int CG, int W>
__device__ __forceinline__ int tile_partial_off(const SeqTiles& st, int qt, int H_q) {
  // full tiles below qt (all full tiles, for the partial last tile)
  const int below = (st.partial && qt == st.n_tiles - 1) ? st.n_full : qt;
  int off = 0;
  full_runs<W>(st, [&](int lo, int hi, int k) {
    const int top = min(hi, below - 1);
    if (k > 1 && top >= lo) off += (top - lo + 1) * 16 * H_q * k;
    return false;
  });
  return off;
}

// Items of one sequence; its weight: the key tiles of its heaviest chunk
// (the top tile's), the order in which batches of up to kRankSeqs sequences
// deal their items; and its partial rows (P_b above: 0 if it does not split).
template <int CG, int W>
__device__ __forceinline__ int seq_items(const SeqInfo& s, const SeqTiles& st, int G, int H_q,
                                         int& weight, int& prows) {
  int n = 0;
  weight = 0;
  prows = 0;
  if (st.n_tiles <= 0) return 0;
  const TilePlan top = tile_plan<CG, W>(st.n_tiles - 1, s, G);
  weight = (top.n_ktiles + top.n_chunks - 1) / top.n_chunks;
  if (st.n_tiles == 1 && top.n_ctiles == 1) {  // one narrow tile (a decode row)
    if (CIE_MIXED_NARROW_ORDER == 1) weight = 0;
    if (CIE_MIXED_NARROW_ORDER == 2) weight += 1 << 24;
  }
  if (st.partial) {
    n += top.n_groups * top.n_chunks;
    if (top.n_chunks > 1) prows += top.rows * H_q * top.n_chunks;
  }
  const int ng = st.ng_full;
  full_runs<W>(st, [&](int lo, int hi, int k) {
    n += (hi - lo + 1) * ng * k;
    if (k > 1) prows += (hi - lo + 1) * 16 * H_q * k;
    return false;
  });
  return n;
}

// Item j of one sequence: its query tile and its index among the tile's
// items (column group * chunks + chunk).
template <int CG, int W>
__device__ __forceinline__ void seq_locate(const SeqInfo& s, const SeqTiles& st, int G, int j,
                                           int& qt, int& jt) {
  qt = st.n_tiles - 1;
  jt = j;
  if (st.partial) {
    const TilePlan tp = tile_plan<CG, W>(st.n_tiles - 1, s, G);
    const int np = tp.n_groups * tp.n_chunks;
    if (j < np) return;
    j -= np;
  }
  const int ng = st.ng_full;
  full_runs<W>(st, [&](int lo, int hi, int k) {
    const int per = ng * k;
    const int cnt = (hi - lo + 1) * per;
    if (j < cnt) {
      const int d = j / per;
      qt = hi - d;
      jt = j - d * per;
      return true;
    }
    j -= cnt;
    return false;
  });
}

// Inclusive sum of (x, y) over the workgroup's first `span` threads (sm: NTH
// int2; rounds only as many as span needs).
template <int NTH>
__device__ __forceinline__ int2 block_scan2(int2 v, int2* sm, int span) {
  sm[threadIdx.x] = v;
  __syncthreads();
  for (int off = 1; off < span; off <<= 1) {
    const int2 add = threadIdx.x >= (unsigned)off ? sm[threadIdx.x - off] : int2{0, 0};
    __syncthreads();
    v.x += add.x;
    v.y += add.y;
    sm[threadIdx.x] = v;
    __syncthreads();
  }
  return v;
}

// Last index i in [0, n) with prefix[i] <= x (prefix nondecreasing,
// prefix[0] <= x): i + 1 such entries, counted 64 per LDS read with a ballot.
__device__ __forceinline__ int prefix_search(const int* prefix, int n, int x) {
  int n_le = 0;
  // (the lane's address derived afresh: hoisted out of the item loop, it
  // would hold a register through every key loop)
  const int* const mine = prefix + (opaque((int)threadIdx.x) & (kWave - 1));
  for (int i0 = 0; i0 < n; i0 += kWave) {
    const int i = i0 + (int)(threadIdx.x & (kWave - 1));
    const uint64_t le = __ballot(i < n && mine[i0] <= x);
    n_le += __popcll(le);
    if (~le != 0) break;
  }
  return uniform(n_le - 1);
}

// One work item: column group gi, chunk `chunk` of query tile qt of sequence
// b, kv head g.
template <int D, bool P32>
__device__ __forceinline__ void process_item(const MixedParams& p, const SeqInfo& s, int b, int g,
                                             int qt, int j, f32x4* sm_facc, float2* sm_fml,
                                             f16x8* sm_q, int* sm_last, int item) {
  constexpr int CG = col_group<D>();
  constexpr int W = mixed_waves<D>();
  const int tid = opaque((int)threadIdx.x);
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const int r16 = lane & 15;
  const int grp = lane >> 4;
  TilePlan tp = tile_plan<CG, W>(qt, s, p.G);
  // the block's base, taken once here, where the key loop's registers are
  // not yet live (after the loop, the run walk it takes spills scalars)
  if (tp.n_chunks > 1)
    tp.pblk = s.L <= 16 ? s.pbase  // one tile
                        : uniform(s.pbase + tile_partial_off<CG, W>(seq_tiles<CG, W>(s, p.n_qtiles, p.G),
                                                                    qt, p.H_q));
  const int gi = j / tp.n_chunks;
  const int chunk = j - gi * tp.n_chunks;
  const int ct0 = gi * tp.cg;
  const int n = min(tp.cg, tp.n_ctiles - ct0);
  // this chunk's key tiles, and this wave's share of them
  int kt0, kt1, w0, w1;
  split_steps(0, tp.n_ktiles, chunk, tp.n_chunks, kt0, kt1);
  split_steps_front(kt0, kt1, wave, W, w0, w1);
  const PagedSrc src{p.k_pool,  p.v_pool,  p.block_table + s.slot * p.bt_stride,
                     (int64_t)g * p.pool_head_stride, p.pool_page_stride, p.n_pages,
                     p.page_size, p.err, p.tpp_magic, p.pool_bytes};
  switch (n) {
#define CIE_GROUP_CASE(k)                                                                      \
  case k:                                                                                      \
    if constexpr (k <= CG)                                                                     \
      run_group<D, P32, k>(p, s, tp, g, ct0, chunk, w0, w1, src, wave, r16, grp, sm_facc,     \
                           sm_fml, sm_q, item);                                               \
    break;
    CIE_GROUP_CASE(1)
    CIE_GROUP_CASE(2)
    CIE_GROUP_CASE(3)
    CIE_GROUP_CASE(4)
#undef CIE_GROUP_CASE
    default:
      break;
  }
  MIXED_TRACE(item, 2, __builtin_amdgcn_s_memrealtime());
  MIXED_TRACE(item, 5, (uint64_t)(tp.n_ctiles * 1000000 + tp.n_chunks * 10000 + (kt1 - kt0)));
  // (no barrier before the next item: its first LDS writes, the Q copy,
  // touch nothing the fold reads, and its Q barrier orders the rest)
  if (tp.n_chunks == 1) {
    MIXED_TRACE(item, 3, __builtin_amdgcn_s_memrealtime());
    MIXED_TRACE_FLUSH(g, item);
    return;
  }
  // The last chunk of this (tile, column group) to arrive merges all chunks.
  int32_t* ctr =
      p.counters + (((int64_t)b * p.H_kv + g) * p.n_qtiles + qt) * kMaxColGroups + gi;
  const int64_t n_words = (int64_t)p.B * p.H_kv * p.n_qtiles * kMaxColGroups;
  if (arrive_last(ctr, n_words, tp.n_chunks, sm_last, p.err)) {
    MIXED_TRACE(item, 4, __builtin_amdgcn_s_memrealtime());
    merge_group<D>(p, s, tp, g, ct0, min(16 * n, tp.n_combos - 16 * ct0));
    if (threadIdx.x == 0) counter_reset(ctr);
  }
  MIXED_TRACE(item, 3, __builtin_amdgcn_s_memrealtime());
  MIXED_TRACE_FLUSH(g, item);
}

// Grid: one workgroup per CU, a whole number per kv head (workgroup w serves
// kv head w % H_kv).  Every workgroup plans the whole batch — per sequence
// item counts, the order in which sequences deal their items (heaviest
// first for batches of up to kRankSeqs sequences) and the item prefix by
// that order, in LDS — and takes its kv head's items round by round
// (see the item loop), so no workgroup is launched for an empty slot.
// Waves per SIMD the registers must allow: two when a wave carries at most
// two column tiles or keeps its Q operands in LDS (D = 64), else one.
template <int D>
constexpr int mixed_waves_per_simd() {
  return D <= 64 && (col_group<D>() <= 2 || CIE_MIXED_QLDS) ? 2 : 1;
}

// The kernel's static LDS, element counts of its arrays: the waves' states
// in the fold — [slot][d-tile][lane] (acc) and [slot][lane] (m, l), slot =
// fold_slot(wave, column tile) — the item's Q operands, and the block scan.
template <int D>
struct MixedLds {
  static constexpr int W = mixed_waves<D>();
  static constexpr int kFold = col_group<D>() * (W - 1);
  static constexpr int facc = kFold * Geo<D>::NT * kWave;  // f32x4
  static constexpr int fml = kFold * kWave;                // float2
  static constexpr int q = CIE_MIXED_QLDS ? col_group<D>() * Geo<D>::KS * kWave : 1;  // f16x8
  static constexpr int scan = W * kWave;                   // int2
  static constexpr size_t bytes = facc * sizeof(f32x4) + fml * sizeof(float2) + q * sizeof(f16x8) +
                                  scan * sizeof(int2) + 16 /* sm_last, aligned */;
};
// Every build must be able to plan a batch of kMaxSeqs sequences: its static
// LDS plus the plan tables of kMaxSeqs sequences fit one workgroup's LDS.  (A
// build with 8 waves asked for 170,004 bytes at 1,024 sequences, past the
// 160 KiB a workgroup may have; the launcher's run-time refusal is a second
// line of defence for devices with less.)
template <int D>
constexpr bool mixed_lds_fits() {
  return MixedLds<D>::bytes + mixed_plan_lds(kMaxSeqs) <= kLdsPerWorkgroup;
}

// The batch's plan tables in LDS (sm_plan, mixed_plan_lds(B) bytes), all by
// position in the order in which sequences deal their items: the sequence
// and its seq_info (so an item starts its Q and page-id loads without
// reading the sequence tables again), and the item prefix.
struct PlanTables {
  int2* tp;     // (t0, partial base)
  int* slot;
  int* rows;
  int* prior;
  int* order;   // the sequence at each position
  int* prefix;  // B + 1 entries, by position
  __device__ __forceinline__ PlanTables(char* sm, int B) {
    tp = reinterpret_cast<int2*>(sm);
    slot = reinterpret_cast<int*>(tp + B);
    rows = slot + B;
    prior = rows + B;
    order = prior + B;
    prefix = order + B;
  }
  __device__ __forceinline__ SeqInfo seq(int pos) const {
    SeqInfo s;
    const int2 tb = tp[pos];
    s.t0 = uniform(tb.x);
    s.slot = uniform(slot[pos]);
    s.L = uniform(rows[pos]);
    s.c = uniform(prior[pos]);
    s.pbase = uniform(tb.y);
    return s;
  }
};

// Plans the batch into the tables (every workgroup of an unplanned launch
// does this; a planned launch reads the result from cie_mixed_plan):
// per-sequence item counts, partial bases and the dealing order; returns
// the item count (uniform).
template <int D>
__device__ __forceinline__ int plan_batch(const MixedParams& p, const PlanTables& t, int2* sm_scan) {
  constexpr int W = mixed_waves<D>();
  constexpr int NTH = W * kWave;
  constexpr int CG = col_group<D>();
  const int B = p.B;
  int2* const sm_tp = t.tp;
  int* const sm_slot = t.slot;
  int* const sm_rows = t.rows;
  int* const sm_prior = t.prior;
  int* const sm_order = t.order;
  int* const sm_prefix = t.prefix;
  int base = 0;
  if (B <= kWave) {
    // A batch of up to 64 sequences: every wave plans it alone, a lane per
    // sequence, and writes the same tables (identical values from every
    // wave), reading back only what it wrote itself — no barrier.
    const int lane = threadIdx.x & (kWave - 1);
    int n = 0, key = -1, prows = 0;
    SeqInfo s{0, 0, 0, 0, 0};  // pbase 0: counted as split
    if (lane < B) {
      s = seq_info(p, lane);
      if (blockIdx.x == 0 && threadIdx.x < kWave && ((s.L + 15) >> 4) > p.n_qtiles)
        set_err(p.err, CIE_ERRBIT_LEN);  // rows past max_seqlen are not computed
      int weight = 0;
      if (s.L > 0)
        n = seq_items<CG, W>(s, seq_tiles<CG, W>(s, p.n_qtiles, p.G), p.G, p.H_q, weight, prows);
      key = n > 0 ? weight : -1;
      prows = (int)min((int64_t)prows, p.part_cap + 1);
    }
    // Partial base: the partial rows of the sequences before this one in
    // sequence order (lanes past B count 0).
    const int p_incl = wave_inclusive_sum(prows);
    const int pfx = p_incl - prows;
    const int ptot = __builtin_amdgcn_readlane(p_incl, kWave - 1);
    // Position: heaviest sequence first, ties by b.  Rank keys (key + 1,
    // clamped to 25 bits, above the lane's complement) are distinct, and a
    // larger one comes earlier; lanes past B write 0, which ranks no one.
    // Every lane reads all keys and item counts by broadcast LDS reads and
    // counts the sequences ahead of it and their items: its position and
    // its item prefix in one pass, with no shuffles.
    auto rank_key = [&](int k) {
      return lane < B ? ((uint32_t)min(k + 1, (1 << 25) - 1) << 6) | (uint32_t)(kWave - 1 - lane) : 0u;
    };
    uint32_t rk = rank_key(key);
    uint32_t* const sm_rk = reinterpret_cast<uint32_t*>(sm_scan);  // [kWave]
    int* const sm_rn = reinterpret_cast<int*>(sm_scan) + kWave;     // [kWave]
    sm_rk[lane] = rk;
    sm_rn[lane] = n;
    int pos = 0, before = 0, tot = 0;
    for (int o = 0; o < B; o += 4) {
      const uint4 kk = *reinterpret_cast<const uint4*>(sm_rk + o);
      const int4 nn = *reinterpret_cast<const int4*>(sm_rn + o);
      pos += (int)(kk.x > rk) + (int)(kk.y > rk) + (int)(kk.z > rk) + (int)(kk.w > rk);
      before += (kk.x > rk ? nn.x : 0) + (kk.y > rk ? nn.y : 0) + (kk.z > rk ? nn.z : 0) +
                (kk.w > rk ? nn.w : 0);
      tot += nn.x + nn.y + nn.z + nn.w;
    }
    s.pbase = pfx;
    if (ptot > p.part_cap) {
      // The batch's split tiles need more partial rows than the buffer
      // holds: a sequence whose rows end past it runs unsplit, and the
      // batch is ranked again with its counts — in arrays of their own, as
      // another wave may still be reading the first ones.
      s.pbase = (int64_t)pfx + prows <= p.part_cap ? pfx : -1;
      if (lane < B && s.pbase < 0 && s.L > 0) {
        int weight = 0, unused = 0;
        n = seq_items<CG, W>(s, seq_tiles<CG, W>(s, p.n_qtiles, p.G), p.G, p.H_q, weight, unused);
        key = n > 0 ? weight : -1;
      }
      rk = rank_key(key);
      uint32_t* const sm_rk2 = reinterpret_cast<uint32_t*>(sm_scan) + 2 * kWave;  // [kWave]
      int* const sm_rn2 = reinterpret_cast<int*>(sm_scan) + 3 * kWave;            // [kWave]
      sm_rk2[lane] = rk;
      sm_rn2[lane] = n;
      pos = before = tot = 0;
      for (int o = 0; o < B; o += 4) {
        const uint4 kk = *reinterpret_cast<const uint4*>(sm_rk2 + o);
        const int4 nn = *reinterpret_cast<const int4*>(sm_rn2 + o);
        pos += (int)(kk.x > rk) + (int)(kk.y > rk) + (int)(kk.z > rk) + (int)(kk.w > rk);
        before += (kk.x > rk ? nn.x : 0) + (kk.y > rk ? nn.y : 0) + (kk.z > rk ? nn.z : 0) +
                  (kk.w > rk ? nn.w : 0);
        tot += nn.x + nn.y + nn.z + nn.w;
      }
    }
    if (lane < B) {
      sm_tp[pos] = int2{(int)s.t0, s.pbase};
      sm_slot[pos] = (int)s.slot;
      sm_rows[pos] = s.L;
      sm_prior[pos] = s.c;
      sm_order[pos] = lane;
      sm_prefix[pos + 1] = before + n;
    }
    if (lane == 0) sm_prefix[0] = 0;
    base = tot;
  } else {
    // Larger batches keep their order (position = sequence): per-sequence
    // tables, item counts and partial rows, sequences b = tid, tid + NTH,
    // ... (B <= kMaxSeqs), then a block scan of both: the item prefix and
    // each sequence's partial base.
    for (int b = threadIdx.x; b < B; b += NTH) {
      const SeqInfo s = seq_info(p, b);  // pbase 0: counted as split
      sm_tp[b].x = (int)s.t0;
      sm_slot[b] = (int)s.slot;
      sm_rows[b] = s.L;
      sm_prior[b] = s.c;
      if (blockIdx.x == 0 && ((s.L + 15) >> 4) > p.n_qtiles)
        set_err(p.err, CIE_ERRBIT_LEN);  // rows past max_seqlen are not computed
      int n = 0, weight = 0, prows = 0;
      if (s.L > 0)
        n = seq_items<CG, W>(s, seq_tiles<CG, W>(s, p.n_qtiles, p.G), p.G, p.H_q, weight, prows);
      sm_prefix[b + 1] = n;
      sm_tp[b].y = (int)min((int64_t)prows, p.part_cap + 1);  // the base, after the scan
      sm_order[b] = b;
    }
    __syncthreads();
    int ptot = 0;
    for (int q0 = 0; q0 < B; q0 += NTH) {
      const int q = q0 + threadIdx.x;
      const int2 c = q < B ? int2{sm_prefix[q + 1], sm_tp[q].y} : int2{0, 0};
      const int span = min(NTH, B - q0);
      const int2 inc = block_scan2<NTH>(c, sm_scan, span);
      const int2 tot = sm_scan[span - 1];
      if (q < B) {
        sm_prefix[q + 1] = base + inc.x;
        sm_tp[q].y = ptot + inc.y - c.y;  // exclusive
      }
      base += tot.x;
      ptot += tot.y;
      __syncthreads();
    }
    if (ptot > p.part_cap) {
      // The batch's split tiles need more partial rows than the buffer
      // holds: a sequence whose rows end past it runs unsplit; its item
      // count is taken again and the item prefix scanned again.
      for (int b = threadIdx.x; b < B; b += NTH) {
        SeqInfo s;
        s.t0 = sm_tp[b].x;
        s.slot = sm_slot[b];
        s.L = sm_rows[b];
        s.c = sm_prior[b];
        s.pbase = 0;
        int n = 0, weight = 0, prows = 0;
        if (s.L > 0)
          n = seq_items<CG, W>(s, seq_tiles<CG, W>(s, p.n_qtiles, p.G), p.G, p.H_q, weight, prows);
        const int pb = sm_tp[b].y;
        s.pbase = (int64_t)pb + min((int64_t)prows, p.part_cap + 1) <= p.part_cap ? pb : -1;
        sm_tp[b].y = s.pbase;
        if (s.pbase < 0 && s.L > 0)
          n = seq_items<CG, W>(s, seq_tiles<CG, W>(s, p.n_qtiles, p.G), p.G, p.H_q, weight, prows);
        sm_prefix[b + 1] = n;
      }
      __syncthreads();
      base = 0;
      for (int q0 = 0; q0 < B; q0 += NTH) {
        const int q = q0 + threadIdx.x;
        const int c = q < B ? sm_prefix[q + 1] : 0;
        const int span = min(NTH, B - q0);
        const int2 inc = block_scan2<NTH>(int2{c, 0}, sm_scan, span);
        const int tot = sm_scan[span - 1].x;
        if (q < B) sm_prefix[q + 1] = base + inc.x;
        base += tot;
        __syncthreads();
      }
    }
    if (threadIdx.x == 0) sm_prefix[0] = 0;
    __syncthreads();
  }
  return uniform(base);
}

template <int D, bool P32, bool kPlanned>
__global__ __launch_bounds__(mixed_waves<D>() * kWave)
__attribute__((amdgpu_waves_per_eu(mixed_waves_per_simd<D>()))) void mixed_attention_kernel(
    MixedParams p) {
  static_assert(col_group<D>() <= 4 && 8 / col_group<D>() <= kMaxColGroups, "column groups");
  static_assert(mixed_lds_fits<D>(),
                "static LDS + the plan tables of kMaxSeqs sequences exceed a workgroup's LDS");
  constexpr int W = mixed_waves<D>();
  constexpr int NTH = W * kWave;
  typedef MixedLds<D> Lds;
  __shared__ f32x4 sm_facc[Lds::facc];
  __shared__ float2 sm_fml[Lds::fml];
  __shared__ f16x8 sm_q[Lds::q];
  __shared__ int sm_last;
  // block scan (larger batches); a batch of up to 64 sequences ranks
  // through its first 2 * kWave words
  __shared__ __attribute__((aligned(16))) int2 sm_scan[Lds::scan];
  static_assert(NTH >= kWave && 2 * Lds::scan >= 4 * kWave,
                "rank keys and item counts (and a second ranking) fit the scan buffer");
  // Unplanned launches: the plan tables, in LDS sized by the launch to the
  // batch (mixed_plan_lds).  Planned launches: the descriptors of this
  // workgroup's first kDescRounds items.
  extern __shared__ __attribute__((aligned(16))) char sm_plan[];
  __shared__ __attribute__((aligned(16))) int4 sm_desc[kPlanned ? 2 * kDescRounds : 1];
  const PlanTables tables(sm_plan, p.B);

  constexpr int CG = col_group<D>();
  MIXED_TRACE(0, 15, __builtin_amdgcn_s_memrealtime());  // workgroup start
  const int g = blockIdx.x % p.H_kv;
  const int slot_r = blockIdx.x / p.H_kv;
  const int n_slots_r = gridDim.x / p.H_kv;  // workgroups per kv head
  // item of round q for this workgroup (see the item loop)
  auto item_of = [&](int q) { return q * n_slots_r + ((q & 1) ? n_slots_r - 1 - slot_r : slot_r); };
  int n_items;
  if constexpr (kPlanned) {
    // The step's plan: a header, then one 8-word descriptor per item.  The
    // header and the descriptors of this workgroup's first kDescRounds
    // rounds are loaded together (one memory round trip; a descriptor past
    // the item count is never used), the descriptors into LDS.
    const int32_t* const hdr = p.plan;
    const int tid = threadIdx.x;
    if (tid < 2 * kDescRounds) {
      const int it = item_of(tid >> 1);
      if (it < p.plan_cap)
        sm_desc[tid] = *reinterpret_cast<const int4*>(p.plan + kPlanHeader + (int64_t)it * 8 + 4 * (tid & 1));
    }
    const int4 h0 = *reinterpret_cast<const int4*>(hdr);
    const int4 h1 = *reinterpret_cast<const int4*>(hdr + 4);
    __syncthreads();
    n_items = uniform(h0.x);
    // a plan made for another batch shape, budget or partial layout
    if (uniform(h0.y) != (int)p.part_cap || uniform(h0.z) != p.B || uniform(h0.w) != p.n_qtiles ||
        uniform(h1.x) != p.H_q || uniform(h1.y) != p.H_kv || n_items > p.plan_cap) {
      if (blockIdx.x == 0 && threadIdx.x == 0) set_err(p.err, CIE_ERRBIT_PLAN);
      return;
    }
  } else {
    n_items = plan_batch<D>(p, tables, sm_scan);
  }
  MIXED_TRACE(0, 6, __builtin_amdgcn_s_memrealtime());  // planning done
  MIXED_TRACE(0, 14, (uint64_t)blockIdx.x);

  // Items go to the kv head's workgroups in rounds, alternating direction
  // (round q, position w: item q * n + (q even ? w : n - 1 - w)), so the
  // workgroups that took the heaviest items of round 0 take the lightest of
  // round 1.
  for (int q = 0; slot_r < n_slots_r; ++q) {
    const int item = item_of(q);
    if (item >= n_items) break;
    MIXED_TRACE(item, 0, __builtin_amdgcn_s_memrealtime());
    int b, qt, jt;
    SeqInfo s;
    if constexpr (kPlanned) {
      int4 d0, d1;
      if (q < kDescRounds) {
        d0 = sm_desc[2 * q];
        d1 = sm_desc[2 * q + 1];
      } else {
        d0 = *reinterpret_cast<const int4*>(p.plan + kPlanHeader + (int64_t)item * 8);
        d1 = *reinterpret_cast<const int4*>(p.plan + kPlanHeader + (int64_t)item * 8 + 4);
      }
      b = uniform(d0.x);
      qt = uniform(d0.y);
      jt = uniform(d0.z);
      s.t0 = uniform(d0.w);
      s.slot = uniform(d1.x);
      s.L = uniform(d1.y);
      s.c = uniform(d1.z);
      s.pbase = uniform(d1.w);
    } else {
      const int pos = prefix_search(tables.prefix, p.B, item);
      b = uniform(tables.order[pos]);
      const int j = item - uniform(tables.prefix[pos]);
      s = tables.seq(pos);
      seq_locate<CG, W>(s, seq_tiles<CG, W>(s, p.n_qtiles, p.G), p.G, j, qt, jt);
    }
    MIXED_TRACE(item, 1, __builtin_amdgcn_s_memrealtime());
    MIXED_TRACE(item, 7, (uint64_t)(b * 1000 + qt));
    process_item<D, P32>(p, s, b, g, uniform(qt), uniform(jt), sm_facc, sm_fml, sm_q, &sm_last,
                         item);
  }
}


// A step's plan for its planned mixed launches (cie_mixed_plan): one
// workgroup plans the batch as every workgroup of an unplanned launch does,
// then writes the header {items, partial budget (rows), B, query tiles,
// H_q, H_kv, 0, 0} and, per item in dealing order, its descriptor
// {b, query tile, index in tile, t0, slot, rows, prior, partial base}.
template <int D>
__global__ __launch_bounds__(mixed_waves<D>() * kWave) void mixed_plan_kernel(MixedParams p) {
  constexpr int W = mixed_waves<D>();
  constexpr int NTH = W * kWave;
  constexpr int CG = col_group<D>();
  typedef MixedLds<D> Lds;
  __shared__ __attribute__((aligned(16))) int2 sm_scan[Lds::scan];
  extern __shared__ __attribute__((aligned(16))) char sm_plan[];
  const PlanTables t(sm_plan, p.B);
  const int n_items = plan_batch<D>(p, t, sm_scan);
  __syncthreads();
  int32_t* const out = p.plan_out;
  const bool fits = n_items <= p.plan_cap;
  if (threadIdx.x == 0) {
    // a batch with more items than the capacity (only overlapping
    // sequences can exceed it) gets an empty plan and CIE_ERRBIT_PLAN
    if (!fits) set_err(p.err, CIE_ERRBIT_PLAN);
    *reinterpret_cast<int4*>(out) = int4{fits ? n_items : 0, (int)p.part_cap, p.B, p.n_qtiles};
    *reinterpret_cast<int4*>(out + 4) = int4{p.H_q, p.H_kv, 0, 0};
  }
  if (!fits) return;
  for (int i = threadIdx.x; i < n_items; i += NTH) {
    // the last position whose prefix is at or below i (prefix[0] = 0)
    int lo = 0, hi = p.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (t.prefix[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    const int2 tb = t.tp[lo];
    SeqInfo s;
    s.t0 = tb.x;
    s.slot = t.slot[lo];
    s.L = t.rows[lo];
    s.c = t.prior[lo];
    s.pbase = tb.y;
    int qt, jt;
    seq_locate<CG, W>(s, seq_tiles<CG, W>(s, p.n_qtiles, p.G), p.G, i - t.prefix[lo], qt, jt);
    int32_t* const d = out + kPlanHeader + (int64_t)i * 8;
    *reinterpret_cast<int4*>(d) = int4{t.order[lo], qt, jt, (int)s.t0};
    *reinterpret_cast<int4*>(d + 4) = int4{(int)s.slot, s.L, s.c, s.pbase};
  }
}

// Workgroups of the mixed grid: CIE_MIXED_WG_PER_CU per CU, a whole number
// per kv head.
static int mixed_workgroups(int H_kv) {
  int dev = 0, n_cu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  int per_head = n_cu * CIE_MIXED_WG_PER_CU / H_kv;
  if (per_head < 1) per_head = 1;
  return per_head * H_kv;
}

// LDS a workgroup may use on the current device (160 KiB on gfx950).
static int64_t device_lds_limit() {
  constexpr int kMaxDevices = 64;
  static int64_t lim[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 160 * 1024;
  if (lim[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || n <= 0)
      n = 160 * 1024;
    lim[dev] = n;
  }
  return lim[dev];
}

template <class K>
static int64_t static_lds_of(K kernel) {
  hipFuncAttributes a{};
  return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(kernel)) == hipSuccess
             ? (int64_t)a.sharedSizeBytes
             : 0;
}

template <int D, bool P32, bool kPlanned>
static int64_t mixed_static_lds() {
  static int64_t bytes = -1;
  if (bytes < 0) bytes = static_lds_of(mixed_attention_kernel<D, P32, kPlanned>);
  return bytes;
}

template <int D, bool kPlanned>
static int launch_mixed(const MixedParams& p, hipStream_t stream) {
  dim3 grid(mixed_workgroups(p.H_kv), 1, 1);
  // a batch whose plan tables would take the workgroup past the device's
  // LDS is refused here (the dispatch itself would be rejected); a planned
  // launch reads its plan instead of building the tables
  const size_t dyn = kPlanned ? 0 : mixed_plan_lds(p.B);
  const int64_t lds = (p.pool_bytes != 0 ? mixed_static_lds<D, true, kPlanned>()
                                         : mixed_static_lds<D, false, kPlanned>()) +
                      (int64_t)dyn;
  if (lds > device_lds_limit()) return CIE_EUNSUPPORTED;
  if (p.pool_bytes != 0)
    hipLaunchKernelGGL((mixed_attention_kernel<D, true, kPlanned>), grid,
                       dim3(mixed_waves<D>() * kWave), dyn, stream, p);
  else
    hipLaunchKernelGGL((mixed_attention_kernel<D, false, kPlanned>), grid,
                       dim3(mixed_waves<D>() * kWave), dyn, stream, p);
  return (int)hipGetLastError();
}

template <int D>
static int launch_mixed_plan(const MixedParams& p, hipStream_t stream) {
  static int64_t st = -1;
  if (st < 0) st = static_lds_of(mixed_plan_kernel<D>);
  if (st + (int64_t)mixed_plan_lds(p.B) > device_lds_limit()) return CIE_EUNSUPPORTED;
  hipLaunchKernelGGL((mixed_plan_kernel<D>), dim3(1), dim3(mixed_waves<D>() * kWave),
                     mixed_plan_lds(p.B), stream, p);
  return (int)hipGetLastError();
}

// partials of `rows` rows: part_m | part_l | part_acc, each region 256-byte
// aligned
struct MixedLayout {
  int64_t m, l, acc, total;
};

static MixedLayout mixed_layout(int64_t rows, int64_t D) {
  auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  MixedLayout w;
  w.m = 0;
  w.l = up(rows * 4);
  w.acc = up(w.l + rows * 4);
  w.total = up(w.acc + rows * D * 4);
  return w;
}

// Partial rows a buffer of `bytes` holds (layout total <= bytes).
static int64_t mixed_partial_rows(int64_t bytes, int64_t D) {
  const int64_t r = (bytes - 3 * 256) / (4 * (D + 2));
  return r < 0 ? 0 : (r > kMaxPartRows ? kMaxPartRows : r);
}

// The default budget, per q head: kDefaultRowsPerToken chunk rows per token,
// and at least kMaxChunks rows for each of the first kDefaultChunkedTokens
// tokens.  A decode row (one token) whose keys split into up to kMaxChunks
// chunks needs that many rows; in a batch of mostly decode rows the
// per-token allowance alone would leave most of them unsplit, each row's
// keys streamed by one workgroup (32 rows of 16,384 keys + a 16-token
// prefill: 101.8 us at 2 rows per token, 56.9 at 16).
constexpr int64_t kDefaultRowsPerToken = 2;
constexpr int64_t kDefaultChunkedTokens = 64;

}  // namespace cie

using namespace cie;

extern "C" int64_t cie_mixed_partials_bytes(int64_t total_T, int64_t H_q, int64_t D) {
  if (total_T < 0 || H_q <= 0 || D <= 0 || total_T > ((int64_t)1 << 40) / H_q) return -1;
  const int64_t per_token = kDefaultRowsPerToken * total_T;
  const int64_t chunked = kMaxChunks * (total_T < kDefaultChunkedTokens ? total_T : kDefaultChunkedTokens);
  int64_t rows = (per_token > chunked ? per_token : chunked) * H_q;
  if (rows > kMaxPartRows) rows = kMaxPartRows;
  return mixed_layout(rows, D).total;
}

extern "C" int64_t cie_mixed_counters(int64_t B, int64_t H_kv, int64_t max_seqlen) {
  if (B < 0 || H_kv <= 0 || max_seqlen < 0) return -1;
  // arrival words, then as many stale words (arrive_last)
  return 2 * B * H_kv * ((max_seqlen + 15) / 16) * kMaxColGroups;
}

#ifdef CIE_MIXED_TRACE
// Trace builds only: where the mixed kernel stamps its phases (device buffer
// of 16 uint64 per (kv head, item); NULL turns the stamps off).
extern "C" int cie_mixed_trace_buffer(void* buf) {
  uint64_t* p = static_cast<uint64_t*>(buf);
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_mixed_trace), &p, sizeof(p));
}
#endif

// Checks of the batch shape shared by the entry points, and the parameters
// they determine (the budget of partial rows from partials_bytes included).
static int mixed_shape(MixedParams& p, int64_t B, int64_t total_T, int64_t max_seqlen, int64_t H_q,
                       int64_t H_kv, int64_t D, int64_t page_size, int64_t bt_width,
                       int64_t n_slots, int64_t partials_bytes) {
  if (B < 0 || total_T < 0 || max_seqlen < 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 ||
      bt_width <= 0 || n_slots <= 0 || page_size <= 0 || partials_bytes < 0)
    return CIE_EINVAL;
  const int64_t G = H_q / H_kv;
  const int64_t n_qtiles = (max_seqlen + 15) / 16;
  // item indices (<= total_T tiles x groups x chunks), a sequence's partial
  // rows (<= its tokens x H_q x kMaxChunks) and a tile's partial region (16 *
  // H_q rows of kMaxChunks * D floats) must fit in 31 bits
  if (G > 8 || page_size % 16 != 0 || B > kMaxSeqs || H_kv > 65535 || H_q > 65535 ||
      n_qtiles > 0x7fffffff || bt_width * page_size > 0x7fffffff ||
      (bt_width * page_size / 16) * (page_size / 16) > 0x7fffffff ||  // magic_div of tile ids
      total_T * kMaxColGroups * kMaxChunks > 0x7fffffff ||
      total_T * H_q * kMaxChunks > 0x7fffffff ||
      16 * H_q * kMaxChunks * D * 4 > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  if (D != 64 && D != 128) return CIE_EUNSUPPORTED;
  p.total_T = total_T;
  p.bt_width = (int32_t)bt_width;
  p.n_slots = (int32_t)(n_slots > 0x7fffffff ? 0x7fffffff : n_slots);
  p.B = (int32_t)B;
  p.H_q = (int32_t)H_q;
  p.H_kv = (int32_t)H_kv;
  p.G = (int32_t)G;
  p.page_size = (int32_t)page_size;
  p.n_qtiles = (int32_t)n_qtiles;
  p.g_magic = div_magic((uint32_t)G);
  p.tpp_magic = div_magic((uint32_t)(page_size / 16));
  p.scale_log2 = kLog2e / __builtin_sqrtf((float)D);
  // The buffer sets the budget of partial rows: sequences whose split tiles
  // do not fit run unsplit (the plan's pbase).
  p.part_cap = mixed_partial_rows(partials_bytes, D);
  return CIE_OK;
}

// Items a batch can have at most (the plan's capacity): every sequence's
// query tiles (at most total_T / 16 + B over the batch), each in at most
// kMaxColGroups column groups of kMaxChunks chunks.
static int64_t mixed_plan_items(int64_t B, int64_t total_T) {
  const int64_t n = ((total_T + 15) / 16 + B) * kMaxColGroups * kMaxChunks;
  const int64_t lim = (0x7fffffff - kPlanHeader) / 8;
  return n < lim ? n : lim;
}

// The pointers and pool geometry of an attention launch (planned or not).
static int mixed_operands(MixedParams& p, void* o, const void* q, const void* k_pool,
                          const void* v_pool, const int64_t* block_table, void* partials,
                          int64_t partials_bytes, int32_t* counters, int64_t D, int64_t n_pages,
                          int64_t pool_page_stride, int64_t pool_head_stride, int64_t bt_stride,
                          int64_t bt_width) {
  if (n_pages <= 0 || bt_stride < bt_width) return CIE_EINVAL;
  if (!o || !q || !k_pool || !v_pool || !block_table || (!partials && partials_bytes > 0) ||
      !counters)
    return CIE_EINVAL;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(o) |
       reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool) |
       reinterpret_cast<uintptr_t>(partials) | reinterpret_cast<uintptr_t>(counters)) & 15)
    return CIE_EINVAL;
  if (pool_page_stride % 8 != 0 || pool_head_stride % 8 != 0) return CIE_EINVAL;
  p.o = static_cast<f16*>(o);
  p.q = static_cast<const f16*>(q);
  p.k_pool = static_cast<const f16*>(k_pool);
  p.v_pool = static_cast<const f16*>(v_pool);
  p.block_table = block_table;
  const MixedLayout w = mixed_layout(p.part_cap, D);
  char* ws = static_cast<char*>(partials);
  p.part_m = reinterpret_cast<float*>(ws + w.m);
  p.part_l = reinterpret_cast<float*>(ws + w.l);
  p.part_acc = reinterpret_cast<float*>(ws + w.acc);
  p.counters = counters;
  p.pool_page_stride = pool_page_stride;
  p.pool_head_stride = pool_head_stride;
  p.bt_stride = bt_stride;
  p.n_pages = n_pages;
  const int64_t pool_bytes = n_pages * pool_page_stride * 2;
  p.pool_bytes = pool_bytes < ((int64_t)1 << 32) ? (uint32_t)pool_bytes : 0u;
  return CIE_OK;
}

extern "C" int cie_mixed_attention(void* o, const void* q, const void* k_pool, const void* v_pool,
                                   const int64_t* cu_seqlens, const int64_t* kv_lens,
                                   const int64_t* slot_ids, const int64_t* block_table,
                                   void* partials, int64_t partials_bytes, int32_t* counters,
                                   int64_t B, int64_t total_T,
                                   int64_t max_seqlen, int64_t H_q, int64_t H_kv, int64_t D,
                                   int64_t page_size, int64_t n_pages, int64_t pool_page_stride,
                                   int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
                                   int64_t n_slots, int32_t* err, void* stream) {
  MixedParams p{};
  int rc = mixed_shape(p, B, total_T, max_seqlen, H_q, H_kv, D, page_size, bt_width, n_slots,
                       partials_bytes);
  if (rc == CIE_EINVAL) return rc;
  if (n_pages <= 0 || bt_stride < bt_width) return CIE_EINVAL;
  if (B == 0 || total_T == 0 || max_seqlen == 0) return CIE_OK;
  if (rc != CIE_OK) return rc;
  if (!cu_seqlens || !kv_lens || !slot_ids) return CIE_EINVAL;
  rc = mixed_operands(p, o, q, k_pool, v_pool, block_table, partials, partials_bytes, counters, D,
                      n_pages, pool_page_stride, pool_head_stride, bt_stride, bt_width);
  if (rc != CIE_OK) return rc;
  p.cu_seqlens = cu_seqlens;
  p.kv_lens = kv_lens;
  p.slot_ids = slot_ids;
  p.err = err;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_mixed<64, false>(p, st) : launch_mixed<128, false>(p, st);
}

extern "C" int64_t cie_mixed_plan_bytes(int64_t B, int64_t total_T) {
  if (B < 0 || total_T < 0 || B > kMaxSeqs || total_T > 0x7fffffff) return -1;
  return (kPlanHeader + 8 * mixed_plan_items(B, total_T)) * (int64_t)sizeof(int32_t);
}

extern "C" int cie_mixed_plan(int32_t* plan, int64_t plan_bytes, const int64_t* cu_seqlens,
                              const int64_t* kv_lens, const int64_t* slot_ids, int64_t B,
                              int64_t total_T, int64_t max_seqlen, int64_t H_q, int64_t H_kv,
                              int64_t D, int64_t page_size, int64_t bt_width, int64_t n_slots,
                              int64_t partials_bytes, int32_t* err, void* stream) {
  MixedParams p{};
  int rc = mixed_shape(p, B, total_T, max_seqlen, H_q, H_kv, D, page_size, bt_width, n_slots,
                       partials_bytes);
  if (rc == CIE_EINVAL) return rc;
  if (B == 0 || total_T == 0 || max_seqlen == 0) return CIE_OK;  // the planned call does nothing
  if (rc != CIE_OK) return rc;
  if (!plan || !cu_seqlens || !kv_lens || !slot_ids || (reinterpret_cast<uintptr_t>(plan) & 15) ||
      plan_bytes < cie_mixed_plan_bytes(B, total_T))
    return CIE_EINVAL;
  p.cu_seqlens = cu_seqlens;
  p.kv_lens = kv_lens;
  p.slot_ids = slot_ids;
  p.plan_out = plan;
  p.plan_cap = (int32_t)mixed_plan_items(B, total_T);
  p.err = err;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_mixed_plan<64>(p, st) : launch_mixed_plan<128>(p, st);
}

extern "C" int cie_mixed_attention_planned(void* o, const void* q, const void* k_pool,
                                           const void* v_pool, const int32_t* plan,
                                           int64_t plan_bytes, const int64_t* block_table,
                                           void* partials, int64_t partials_bytes,
                                           int32_t* counters, int64_t B, int64_t total_T,
                                           int64_t max_seqlen, int64_t H_q, int64_t H_kv,
                                           int64_t D, int64_t page_size, int64_t n_pages,
                                           int64_t pool_page_stride, int64_t pool_head_stride,
                                           int64_t bt_stride, int64_t bt_width, int64_t n_slots,
                                           int32_t* err, void* stream) {
  MixedParams p{};
  int rc = mixed_shape(p, B, total_T, max_seqlen, H_q, H_kv, D, page_size, bt_width, n_slots,
                       partials_bytes);
  if (rc == CIE_EINVAL) return rc;
  if (n_pages <= 0 || bt_stride < bt_width) return CIE_EINVAL;
  if (B == 0 || total_T == 0 || max_seqlen == 0) return CIE_OK;
  if (rc != CIE_OK) return rc;
  if (!plan || (reinterpret_cast<uintptr_t>(plan) & 15) ||
      plan_bytes < cie_mixed_plan_bytes(B, total_T))
    return CIE_EINVAL;
  rc = mixed_operands(p, o, q, k_pool, v_pool, block_table, partials, partials_bytes, counters, D,
                      n_pages, pool_page_stride, pool_head_stride, bt_stride, bt_width);
  if (rc != CIE_OK) return rc;
  p.plan = plan;
  p.plan_cap = (int32_t)mixed_plan_items(B, total_T);
  p.err = err;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_mixed<64, true>(p, st) : launch_mixed<128, true>(p, st);
}
