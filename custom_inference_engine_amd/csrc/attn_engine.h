// Wave-level paged attention engine shared by the decode and mixed kernels.
//
// Both kernels run the same inner step on one 64-lane wavefront: stream two
// 16-key tiles (32 keys) of one kv head out of the paged pool, score them
// against up to 16 query columns with MFMA, update an online softmax, and
// accumulate P.V with MFMA.
//
// Layout (v_mfma_f32_16x16x32_f16; lane l, r16 = l % 16, grp = l / 16):
//   S^T = K . Q^T      A = K tile   : lane holds K[key r16][8*grp + 32*ks .. +7]
//                      B = Q^T      : lane holds Q[col r16][8*grp + 32*ks .. +7]
//                      D = S^T      : lane holds S[col r16][key 4*grp + r], r<4
//   O^T = V^T . P^T    B = P^T      : lane holds P[col r16][key(grp, e)], e<8
//                      A = V^T      : lane holds V[key(grp, e)][NT*r16 + nt]
//                      D = O^T      : lane holds O[col r16][NT*(4*grp + r) + nt]
// with key(grp, e) = 16*(e / 4) + 4*grp + e % 4 across the two tiles.  The
// scores an MFMA leaves in a lane are exactly the probabilities that lane must
// feed to the P.V MFMA, so softmax needs no data movement, and every lane's
// V operand comes from 8-byte loads of whole V rows (the sixteen lanes of a
// group read one contiguous 2*D-byte row), so V needs no transpose through LDS.
// One "column" is a query head (decode) or a (query row, head) pair (mixed);
// the G heads that share a kv head reuse every K/V byte inside the MFMA.
//
// Online softmax runs in the exp2 domain (scores pre-scaled by
// D^-0.5 * log2(e)); P is rounded to fp16 for the P.V product and accumulated
// in fp32, as kernels/decode_attention.py:130-139 does with tl.exp / tl.dot.
#pragma once

#include "cie_common.h"

namespace cie {

template <int D>
struct Geo {
  static_assert(D % 32 == 0 && D >= 32 && D <= 128, "head_dim must be 32, 64, 96 or 128");
  static constexpr int KS = D / 32;  // k-steps of the Q.K^T MFMA
  static constexpr int NT = D / 16;  // 16-wide d-tiles of the P.V MFMA
};

template <int N>
struct HVec {
  typedef f16 type __attribute__((ext_vector_type(N)));
};

// Register-staged K/V for two consecutive 16-key tiles.
template <int D>
struct KVPair {
  f16x8 k[2][Geo<D>::KS];
  typename HVec<Geo<D>::NT>::type v[8];
};

// Physical location of a 16-key tile: pool element offset of its first row
// (page and head applied).  Tile index kt covers keys [16*kt, 16*kt + 16).
// page_size is a multiple of 16, so a tile never straddles a page.
struct TileLoc {
  int64_t base;
};

__device__ __forceinline__ TileLoc tile_loc(const int64_t* __restrict__ bt_row, int kt,
                                            int page_size, int64_t n_pages,
                                            int64_t page_stride, int64_t head_off,
                                            int D, int32_t* err) {
  const int tok = kt * 16;
  const int lp = tok / page_size;
  const int off = tok - lp * page_size;
  int64_t page = bt_row[lp];
  if (page < 0 || page >= n_pages) {
    set_err(err, CIE_ERRBIT_PAGE);
    page = 0;
  }
  return TileLoc{page * page_stride + head_off + (int64_t)off * D};
}

// Loads of a step's two tiles (V rows non-temporal: a call reads each once).
// Both tiles are always loaded (a caller with only one tile passes it twice
// and masks the copy with key kNoKey), so every step issues the same loads
// and the compiler can wait for exactly the oldest step in flight instead of
// draining all loads.
template <int D>
__device__ __forceinline__ void load_pair(KVPair<D>& kv, const f16* __restrict__ kpool,
                                          const f16* __restrict__ vpool, TileLoc t0,
                                          TileLoc t1, int r16, int grp) {
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  typedef typename HVec<NT>::type vrow_t;
  const f16* k0 = kpool + t0.base + r16 * D + 8 * grp;
  const f16* v0 = vpool + t0.base + (4 * grp) * D + NT * r16;
  const f16* k1 = kpool + t1.base + r16 * D + 8 * grp;
  const f16* v1 = vpool + t1.base + (4 * grp) * D + NT * r16;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kv.k[0][ks] = *reinterpret_cast<const f16x8*>(k0 + 32 * ks);
#pragma unroll
  for (int e = 0; e < 4; ++e) kv.v[e] = stream_load(reinterpret_cast<const vrow_t*>(v0 + e * D));
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kv.k[1][ks] = *reinterpret_cast<const f16x8*>(k1 + 32 * ks);
#pragma unroll
  for (int e = 0; e < 4; ++e) kv.v[4 + e] = stream_load(reinterpret_cast<const vrow_t*>(v1 + e * D));
}

// A 16-key tile as a raw buffer: descriptor base = the tile's first row
// (page, head and in-page offset applied; built with scalar ops from
// wave-uniform values), num_records = its valid rows.  Loads past the valid
// rows return 0 without touching memory, so rows at or past a sequence's end
// read as zeros (the reference's masked loads) and an absent tile (0 rows)
// costs no memory traffic.  The descriptor is per tile, so pools of any size
// are addressed with 32-bit in-tile offsets.
// All arguments must be wave-uniform (they are pinned to scalar registers
// here so the descriptor never needs a per-lane loop).
template <int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const f16* pool, int64_t elem_off,
                                                           int valid_rows) {
  const uint64_t a = reinterpret_cast<uint64_t>(pool + elem_off);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const int bytes = __builtin_amdgcn_readfirstlane(valid_rows * D * (int)sizeof(f16));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0,
                                           bytes, kBufRsrcWord3);
}

// Per-lane byte offsets inside a tile of the K and V operands (loop
// invariants): K[key r16][8*grp + 32*ks ..] and V[key 4*grp + e][NT*r16 ..].
template <int D>
struct TileLaneOffsets {
  uint32_t k, v;
  __device__ __forceinline__ TileLaneOffsets(int r16, int grp)
      : k((uint32_t)((r16 * D + 8 * grp) * sizeof(f16))),
        v((uint32_t)((4 * grp * D + Geo<D>::NT * r16) * sizeof(f16))) {}
};

// Cache-policy operand of a raw buffer load: nt (non-temporal, not kept for
// reuse).
constexpr int kBufNt = 2;

// VPOL: cache policy of the V loads (kBufNt for rows read once: a stream
// that no other work item reads again).
template <int D, int VPOL = 0>
__device__ __forceinline__ void load_tile_buf(f16x8 (&k)[Geo<D>::KS],
                                              typename HVec<Geo<D>::NT>::type (&v)[4],
                                              __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                              const TileLaneOffsets<D>& lo) {
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  typedef typename HVec<NT>::type vrow_t;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    k[ks] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, lo.k + 64 * ks, 0, 0));
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (NT == 4)
      v[e] = __builtin_bit_cast(vrow_t, __builtin_amdgcn_raw_buffer_load_b64(rv, lo.v + e * D * 2, 0, VPOL));
    else
      v[e] = __builtin_bit_cast(vrow_t, __builtin_amdgcn_raw_buffer_load_b128(rv, lo.v + e * D * 2, 0, VPOL));
  }
}

// Zero the V rows at keys >= key_end (the masked loads of the reference read
// 0 there; pool memory past a sequence's end may hold anything).  key0a /
// key0b: first key of the pair's two tiles (kNoKey: a masked copy).  A step
// whose keys all lie below key_end needs no zeroing: a masked copy of a valid
// tile holds finite values and gets probability 0.
template <int D>
__device__ __forceinline__ void zero_tail_rows(KVPair<D>& kv, int key0a, int key0b, int key_end,
                                               int grp) {
  typedef typename HVec<Geo<D>::NT>::type vrow_t;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = (e < 4 ? key0a : key0b) + 4 * grp + (e & 3);
    if (key >= key_end) kv.v[e] = vrow_t{};
  }
}

// Reference max of a column that has seen no key: finite, so 2^(s - m) of a
// masked score (s = -inf) is 0 with no special case, and any real score
// exceeds the rescale threshold.  A state that saw no key keeps m = kEmptyMax,
// l = 0, acc = 0; folds and merges weight it by 2^(kEmptyMax - M) = 0 (or, if
// every state is empty, sum zeros and write 0).
constexpr float kEmptyMax = -1e30f;

// Online-softmax state for NCT 16-wide column tiles held by one wave.
template <int D, int NCT>
struct SoftmaxAcc {
  float m[NCT];     // reference max (log2 domain), identical across a column's 4 lanes
  float thr[NCT];   // raw score above which m must move: (m + kRescaleSlack) / scale
  f32x4 lsum[NCT];  // [0]: the column's sum of P (an MFMA against ones: no lane reduction)
  float lpart[NCT];  // or: this lane's part of that sum (the pipelined stream; 4 lanes a column)
  f32x4 acc[NCT][Geo<D>::NT];

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      m[c] = kEmptyMax;
      thr[c] = kEmptyMax;
      lsum[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      lpart[c] = 0.f;
#pragma unroll
      for (int nt = 0; nt < Geo<D>::NT; ++nt) acc[c][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // One of the two sums stays zero (constant-folded away by the compiler).
  __device__ __forceinline__ float l(int c) const { return lsum[c][0] + col_sum4(lpart[c]); }
};

// The reference max of a column moves only when a step's max exceeds it by
// more than kRescaleSlack (log2 units), so P = 2^(s - m) stays <= 2^slack
// (exact in fp16, far from overflow in fp32) and the accumulator rescale is
// rare.  o = acc / l does not depend on which reference max is used.
constexpr float kRescaleSlack = 8.f;

// One 32-key step for NCT column tiles.  key0a / key0b = absolute index of the
// first key of the pair's two tiles (the tiles need not be adjacent; an absent
// second tile passes kNoKey).  A column attends key j iff j < lim[c] (per
// lane: causal / length limit of the lane's column); mask_from (wave-uniform)
// is the smallest limit of any column, so steps whose keys all lie below it
// skip the masking.
//
// The column tiles go in batches of up to kAttendBatch; a batch runs in
// phases — its Q.K^T MFMAs, each lane's maximum of its raw scores against the
// column's threshold, one (rare) reference-max update with accumulator
// rescale, its exponentials, its P.V MFMAs and the P.1 MFMA that accumulates
// the row sums — with no branch inside a phase, so one wave overlaps a column
// tile's VALU work with the MFMAs of the others.  The common step needs no
// cross-lane column maximum: a lane compares its own maximum with the
// threshold (the scale is positive), and only the rare update reduces the
// column (col_max4).  exp2 takes fma(s, scale, -m).
#ifndef CIE_ATTEND_BATCH
#define CIE_ATTEND_BATCH 2
#endif
constexpr int kAttendBatch = CIE_ATTEND_BATCH;

// Where a step reads the Q^T operands of its column tiles: registers
// (QRegs) or this wave's LDS block (QLds: one 16-byte slot per (column tile,
// k-step, lane), so a read is one conflict-free ds_read_b128).
template <int D, int NCT>
struct QRegs {
  const f16x8 (&q)[NCT][Geo<D>::KS];
  __device__ __forceinline__ f16x8 operator()(int c, int ks) const { return q[c][ks]; }
};
template <int D>
struct QLds {
  const f16x8* base;  // [column tile][k-step][lane]
  int lane;
  __device__ __forceinline__ f16x8 operator()(int c, int ks) const {
    return base[(c * Geo<D>::KS + ks) * kWave + lane];
  }
};

template <int D, int NCT, bool MASK, class QS>
__device__ __forceinline__ void attend_pair_body(SoftmaxAcc<D, NCT>& st, const KVPair<D>& kv,
                                                 const QS& qop, int key0a,
                                                 int key0b, const int (&lim)[NCT],
                                                 float scale_log2, int grp) {
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  constexpr int SB = NCT < kAttendBatch ? NCT : kAttendBatch;
  f16x8 va[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int e = 0; e < 8; ++e) va[nt][e] = kv.v[e][nt];
  const f16x8 ones = {(f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f};

#pragma unroll
  for (int c0 = 0; c0 < NCT; c0 += SB) {
    f32x4 s[SB][2];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (c0 + i < NCT) {
        s[i][0] = f32x4{0.f, 0.f, 0.f, 0.f};
        s[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const f16x8 qk = qop(c0 + i, ks);
          s[i][0] = mfma16x16x32(kv.k[0][ks], qk, s[i][0]);
          s[i][1] = mfma16x16x32(kv.k[1][ks], qk, s[i][1]);
        }
      }
    }
    float sc[SB][8];
    float xb[SB];  // the lane's maximum raw score per column tile
    bool need = false;
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (c0 + i < NCT) {
        const int c = c0 + i;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[i][r] = s[i][0][r];
          sc[i][4 + r] = s[i][1][r];
        }
        if constexpr (MASK) {
          const int kba = key0a + 4 * grp;
          const int kbb = key0b + 4 * grp;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sc[i][r] = kba + r < lim[c] ? sc[i][r] : kNegInf;
            sc[i][4 + r] = kbb + r < lim[c] ? sc[i][4 + r] : kNegInf;
          }
        }
        xb[i] = fmaxf(fmaxf(fmaxf(sc[i][0], sc[i][1]), fmaxf(sc[i][2], sc[i][3])),
                      fmaxf(fmaxf(sc[i][4], sc[i][5]), fmaxf(sc[i][6], sc[i][7])));
        need |= xb[i] > st.thr[c];
      }
    }
    if (__any(need)) {  // rare: move the reference max, rescale the state
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        if (c0 + i < NCT) {
          const int c = c0 + i;
          const float m_new = fmaxf(st.m[c], col_max4(xb[i]) * scale_log2);
          const float alpha = fast_exp2(st.m[c] - m_new);  // 0 for an empty state
          st.m[c] = m_new;
          st.thr[c] = (m_new + kRescaleSlack) / scale_log2;
          st.lsum[c][0] *= alpha;
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) st.acc[c][nt] *= alpha;
        }
      }
    }
    f16x8 pop[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (c0 + i < NCT) {
        const float m = st.m[c0 + i];
#pragma unroll
        for (int e = 0; e < 8; ++e) pop[i][e] = (f16)fast_exp2(__builtin_fmaf(sc[i][e], scale_log2, -m));
      }
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (c0 + i < NCT) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          st.acc[c0 + i][nt] = mfma16x16x32(va[nt], pop[i], st.acc[c0 + i][nt]);
        st.lsum[c0 + i] = mfma16x16x32(ones, pop[i], st.lsum[c0 + i]);
      }
    }
  }
}

template <int D, int NCT, class QS>
__device__ __forceinline__ void attend_pair(SoftmaxAcc<D, NCT>& st, const KVPair<D>& kv,
                                            const QS& qop, int key0a,
                                            int key0b, const int (&lim)[NCT], int mask_from,
                                            float scale_log2, int grp) {
  if (max(key0a, key0b) + 16 > mask_from)  // uniform
    attend_pair_body<D, NCT, true, QS>(st, kv, qop, key0a, key0b, lim, scale_log2, grp);
  else
    attend_pair_body<D, NCT, false, QS>(st, kv, qop, key0a, key0b, lim, scale_log2, grp);
}

// Output dim held by (grp, r, nt) of the P.V accumulator.
template <int D>
__device__ __forceinline__ int acc_dim(int grp, int r, int nt) {
  return Geo<D>::NT * (4 * grp + r) + nt;
}

// Where a wave's key tiles live: one kv head of one slot's block-table row.
struct PagedSrc {
  const f16* k_pool;
  const f16* v_pool;
  const int64_t* bt_row;
  int64_t head_off;     // kv head * pool head stride
  int64_t page_stride;  // pool page stride
  int64_t n_pages;
  int page_size;
  int32_t* err;
  uint32_t tpp_magic;   // div_magic(page_size / 16) (the mixed kernel's streams)
  uint32_t pool_bytes;  // each pool's size if under 4 GiB, else 0 (the pipelined stream)
};

// Page id of key tile c0 + lane of a wave's tiles [.., t_end) (0 for lanes past
// t_end; a page id outside the pool is reported and read as page 0).
__device__ __forceinline__ int lane_page_id(const PagedSrc& src, int c0, int t_end, int lane) {
  int page = 0;
  if (lane < min(kWave, t_end - c0)) {
    int64_t pg = src.bt_row[magic_div(c0 + lane, src.tpp_magic)];
    if (pg < 0 || pg >= src.n_pages) {
      set_err(src.err, CIE_ERRBIT_PAGE);
      pg = 0;
    }
    page = (int)pg;
  }
  return page;
}

// ---- Key tiles through one buffer descriptor per pool ----
//
// For pools under 4 GiB (the caller checks): one descriptor per pool, with a
// tile's byte offset as the loads' scalar offset — a step costs two
// v_readlane instead of a descriptor per tile (about 17 scalar instructions
// each, which a lone wave per SIMD pays in issue slots).  Rows past key_end
// are then real pool memory: the streams mask their scores like any key past
// a column's limit and zero their V rows in registers.

template <int D>
struct PoolTiles {
  __amdgpu_buffer_rsrc_t kd, vd;
  const PagedSrc* src;
  int t_end, lane, tpp;
  __device__ __forceinline__ PoolTiles(const PagedSrc& s, int t_end_, int lane_)
      : kd(coherent_rsrc(s.k_pool, s.pool_bytes)), vd(coherent_rsrc(s.v_pool, s.pool_bytes)), src(&s),
        t_end(t_end_), lane(lane_), tpp(s.page_size >> 4) {}
  // Tile c0 + lane of the chunk at c0, or its last tile for lanes past it:
  // lane ka + 1 then always holds a step's second tile (the last tile again
  // when it is missing: its keys masked, its V rows zeroed), with no
  // cross-lane step (the extra page-id loads hit the same lines).
  __device__ __forceinline__ int lane_tile(int c0) const { return c0 + min(lane, t_end - c0 - 1); }
  __device__ __forceinline__ int lane_page(int c0) const {
    int64_t pg = src->bt_row[magic_div(lane_tile(c0), src->tpp_magic)];
    if (pg < 0 || pg >= src->n_pages) {
      set_err(src->err, CIE_ERRBIT_PAGE);
      pg = 0;
    }
    return (int)pg;
  }
  // byte offset in the pool of that tile (page, head and in-page rows)
  __device__ __forceinline__ uint32_t lane_offset(int c0, int page) const {
    const int t = lane_tile(c0);
    const int in_page = t - magic_div(t, src->tpp_magic) * tpp;
    return (uint32_t)(((int64_t)page * src->page_stride + src->head_off + (int64_t)(in_page * 16) * D) * 2);
  }
};

// The chunk of up to 64 tiles at c0: its lane offsets and step bookkeeping.
struct PoolChunk {
  uint32_t toff;
  int c0, n_chunk, n_pairs;
  template <int D>
  __device__ __forceinline__ PoolChunk(const PoolTiles<D>& pool, int c0_, int page)
      : toff(pool.lane_offset(c0_, page)), c0(c0_), n_chunk(min(kWave, pool.t_end - c0_)),
        n_pairs((min(kWave, pool.t_end - c0_) + 1) >> 1) {}
  // The first step that needs masking or V-row zeroing against limit (a key
  // at or past it, or a missing second tile): the condition only grows with
  // the step, so each step tests one scalar instead of recomputing its keys.
  // Step j < n_pairs holds keys [16 * (c0 + 2j), + 32): it qualifies iff
  // 16 * (c0 + 2j) + 32 > limit, or its second tile is missing
  // (2j + 1 == n_chunk).
  __device__ __forceinline__ int first_step_past(int limit) const {
    const int x = limit - 32 - 16 * c0;  // in int range: keys < 2^31 - 32
    int j = x < 0 ? 0 : x / 32 + 1;
    if (n_chunk & 1) j = min(j, n_pairs - 1);
    return uniform(j);
  }
  // byte offsets of step j's two tiles (past the last step: the last step's)
  __device__ __forceinline__ void offsets(int j, uint32_t& oa, uint32_t& ob) const {
    const int ka = 2 * min(j, n_pairs - 1);
    oa = __builtin_amdgcn_readlane(toff, ka);
    ob = __builtin_amdgcn_readlane(toff, ka + 1);
  }
  // first keys of step j's two tiles (kNoKey for a missing second tile)
  __device__ __forceinline__ void step_keys(int j, int& ka, int& kb) const {
    const int a = 2 * min(j, n_pairs - 1);
    ka = (c0 + a) * 16;
    kb = a + 1 < n_chunk ? ka + 16 : kNoKey;
  }
};

// One K load (n < 2 * KS: tile n % 2, k-step n / 2) or V load (n < 8: tile
// n / 4, row 4 * grp + n % 4) of a step whose tile offsets are o; ko / vo:
// the lane's offsets inside a tile (TileLaneOffsets).
template <int D>
__device__ __forceinline__ void pool_load_k(KVPair<D>& kv, __amdgpu_buffer_rsrc_t kd, const uint32_t (&o)[2],
                                            uint32_t ko, int n) {
  const int t = n % 2, ks = n / 2;
  kv.k[t][ks] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(kd, ko + 64 * ks, o[t], 0));
}
template <int D, int VPOL = 0>
__device__ __forceinline__ void pool_load_v(KVPair<D>& kv, __amdgpu_buffer_rsrc_t vd, const uint32_t (&o)[2],
                                            uint32_t vo, int n) {
  typedef typename HVec<Geo<D>::NT>::type vrow_t;
  const int t = n / 4, e = n % 4;
  if constexpr (Geo<D>::NT == 4)
    kv.v[n] = __builtin_bit_cast(vrow_t, __builtin_amdgcn_raw_buffer_load_b64(vd, vo + e * D * 2, o[t], VPOL));
  else
    kv.v[n] = __builtin_bit_cast(vrow_t, __builtin_amdgcn_raw_buffer_load_b128(vd, vo + e * D * 2, o[t], VPOL));
}

// stream_tiles (below) through one descriptor per pool: attend_pair steps of
// one or more column tiles, PF steps of loads in flight; the mixed kernel's
// one-column-tile items (decode rows) run it.
template <int D, int NCT, int PF, class QS, class Prologue, int VPOL = 0>
__device__ __forceinline__ void stream_tiles_pool(SoftmaxAcc<D, NCT>& st, const QS& qop,
                                                  const int (&lim)[NCT], int t_begin, int t_end,
                                                  int key_end, const PagedSrc& src, float scale_log2,
                                                  int r16, int grp, Prologue prologue) {
  t_begin = uniform(t_begin);
  t_end = uniform(t_end);
  key_end = uniform(key_end);
  if (t_begin >= t_end) {
    prologue();
    return;
  }
  int mask_from = kNoKey;
#pragma unroll
  for (int c = 0; c < NCT; ++c) mask_from = min(mask_from, lim[c]);
  // (kept in a vector register, as in stream_tiles)
  for (int off = 1; off < kWave; off <<= 1) mask_from = min(mask_from, __shfl_xor(mask_from, off, kWave));
  const int lane = threadIdx.x & (kWave - 1);
  const TileLaneOffsets<D> lanes(r16, grp);
  const PoolTiles<D> pool(src, t_end, lane);
  const __amdgpu_buffer_rsrc_t k_none = coherent_rsrc(src.k_pool, 0);
  const __amdgpu_buffer_rsrc_t v_none = coherent_rsrc(src.v_pool, 0);
  int page = pool.lane_page(t_begin);
  prologue();  // while the first page ids are in flight
  for (int c0 = t_begin; c0 < t_end; c0 += kWave) {
    if (c0 != t_begin) page = pool.lane_page(c0);
    const PoolChunk ch(pool, c0, page);
    const int j_tail = ch.first_step_past(key_end);
    KVPair<D> ring[PF + 1];
    int keya[PF + 1], keyb[PF + 1];
    // every iteration issues one step's loads, so the wait before a step's
    // math covers that step's loads only; past the last step they go
    // through descriptors of no records (zeros, no memory access)
    auto issue = [&](int slot, int j) {
      uint32_t o[2];
      ch.offsets(j, o[0], o[1]);
      uint32_t ko = lanes.k, vo = lanes.v;
      asm volatile("" : "+v"(ko), "+v"(vo));
      const bool real = j < ch.n_pairs;
      const __amdgpu_buffer_rsrc_t kd = real ? pool.kd : k_none;
      const __amdgpu_buffer_rsrc_t vd = real ? pool.vd : v_none;
#pragma unroll
      for (int n = 0; n < 2 * Geo<D>::KS; ++n) pool_load_k<D>(ring[slot], kd, o, ko, n);
#pragma unroll
      for (int n = 0; n < 8; ++n) pool_load_v<D, VPOL>(ring[slot], vd, o, vo, n);
      ch.step_keys(j, keya[slot], keyb[slot]);
    };
#pragma unroll
    for (int j = 0; j < PF; ++j) issue(j, j);
    for (int j0 = 0; j0 < ch.n_pairs; j0 += PF + 1) {
#pragma unroll
      for (int u = 0; u <= PF; ++u) {
        const int j = j0 + u;
        issue((u + PF) % (PF + 1), j + PF);
        if (j < ch.n_pairs) {
          if (j >= j_tail) zero_tail_rows<D>(ring[u], keya[u], keyb[u], key_end, grp);
          attend_pair<D, NCT, QS>(st, ring[u], qop, keya[u], keyb[u], lim, mask_from, scale_log2, grp);
        }
      }
    }
  }
}

// Stream key tiles [t_begin, t_end) of one wave through attend_pair, two
// tiles per step.  The page ids of up to 64 tiles are gathered first, one per
// lane, so a step's K/V loads depend on no other load; a ring of PF + 1
// register-staged steps keeps PF steps of loads in flight ahead of the math.
// Tiles are read through per-tile buffer descriptors (tile_rsrc), so keys at
// or past key_end read as zeros.
// key_end = number of keys that exist (rows at or past it are zeroed).
// prologue() runs once, after the first page-id loads are issued and before
// any K/V load (or at once when the wave has no tiles): the caller stages
// operands there (its Q), so their loads and the page ids' take one memory
// round trip together.
template <int D, int NCT, int PF, class QS, class Prologue, int VPOL = 0>
__device__ __forceinline__ void stream_tiles(SoftmaxAcc<D, NCT>& st, const QS& qop,
                                             const int (&lim)[NCT], int t_begin, int t_end,
                                             int key_end, const PagedSrc& src, float scale_log2,
                                             int r16, int grp, Prologue prologue) {
  // the bounds are wave-uniform: held in scalar registers, so the per-step
  // tile bookkeeping below is scalar work
  t_begin = uniform(t_begin);
  t_end = uniform(t_end);
  key_end = uniform(key_end);
  if (t_begin >= t_end) {
    prologue();
    return;
  }
  int mask_from = kNoKey;
#pragma unroll
  for (int c = 0; c < NCT; ++c) mask_from = min(mask_from, lim[c]);
  // smallest limit over the wave's columns (wave-uniform; kept in a vector
  // register: as a scalar it splits the masked and unmasked steps into
  // separate paths and the step's registers spill)
  for (int off = 1; off < kWave; off <<= 1) mask_from = min(mask_from, __shfl_xor(mask_from, off, kWave));
  const int lane = threadIdx.x & (kWave - 1);
  const int tpp = src.page_size >> 4;  // 16-key tiles per page
  const TileLaneOffsets<D> lanes(r16, grp);
  // page ids of tiles c0 + lane, one per lane
  auto lane_pages = [&](int c0) { return lane_page_id(src, c0, t_end, lane); };
  // pool element offset of tile c0 + lane (page, head and in-page rows
  // applied), computed once per 64 tiles so a step only reads two lanes
  auto lane_offsets = [&](int c0, int page) {
    const int t = c0 + lane;
    const int in_page = t - magic_div(t, src.tpp_magic) * tpp;
    return (int64_t)page * src.page_stride + src.head_off + (int64_t)(in_page * 16) * D;
  };
  int page = lane_pages(t_begin);
  prologue();  // while the first page ids are in flight
  for (int c0 = t_begin; c0 < t_end; c0 += kWave) {
    const int n_chunk = min(kWave, t_end - c0);
    if (c0 != t_begin) page = lane_pages(c0);
    const int64_t toff = lane_offsets(c0, page);
    const int n_pairs = (n_chunk + 1) >> 1;
    KVPair<D> ring[PF + 1];
    int keya[PF + 1], keyb[PF + 1];
    // Every iteration issues one step's loads (past the last step: tiles
    // with no valid rows, which read zeros and touch no memory), so the wait
    // before a step's math covers that step's loads only.
    auto issue = [&](int slot, int j) {
      const bool real = j < n_pairs;
      j = min(j, n_pairs - 1);
      const int ka = 2 * j;  // chunk-local index of the step's first tile
      const bool two = ka + 1 < n_chunk;
      const int key0a = (c0 + ka) * 16;
      const int rows_a = real ? min(16, max(0, key_end - key0a)) : 0;
      const int rows_b = (real && two) ? min(16, max(0, key_end - key0a - 16)) : 0;
      const int64_t oa = readlane64(toff, ka);
      const int64_t ob = two ? readlane64(toff, ka + 1) : oa;
      typedef typename HVec<Geo<D>::NT>::type vrow_t;
      typedef vrow_t vquad_t[4];
      load_tile_buf<D, VPOL>(ring[slot].k[0], *reinterpret_cast<vquad_t*>(&ring[slot].v[0]),
                             tile_rsrc<D>(src.k_pool, oa, rows_a), tile_rsrc<D>(src.v_pool, oa, rows_a),
                             lanes);
      load_tile_buf<D, VPOL>(ring[slot].k[1], *reinterpret_cast<vquad_t*>(&ring[slot].v[4]),
                             tile_rsrc<D>(src.k_pool, ob, rows_b), tile_rsrc<D>(src.v_pool, ob, rows_b),
                             lanes);
      keya[slot] = key0a;
      keyb[slot] = two ? key0a + 16 : kNoKey;
    };
#pragma unroll
    for (int j = 0; j < PF; ++j) issue(j, j);
    for (int j0 = 0; j0 < n_pairs; j0 += PF + 1) {
#pragma unroll
      for (int u = 0; u <= PF; ++u) {
        const int j = j0 + u;
        issue((u + PF) % (PF + 1), j + PF);
        if (j < n_pairs)
          attend_pair<D, NCT, QS>(st, ring[u], qop, keya[u], keyb[u], lim, mask_from, scale_log2, grp);
      }
    }
  }
}

// ---- The software-pipelined stream (mixed kernel) ----
//
// A wave's 32-key step t is: S(t) = K(t) . Q^T for its column tiles, the
// reference-max check on S(t), then P(t) = 2^(S(t)*scale - m) and
// acc += V(t)^T . P(t)^T.  stream_tiles_pipelined puts step t's softmax and
// P.V and step t+1's S MFMAs in one basic block (they depend on nothing in
// each other), in segments of one column tile each (step_segment); the
// masking and reference-max check of step t+1 follow in their own short
// blocks, the rare rescale in a branch.
//
// The step is VALU-bound on one wave: measured on gfx950 (timing kernels on
// register operands), its 32 MFMAs take ~525 cycles and its softmax VALU
// work alone ~930, half of that the 32 v_exp_f32 (a transcendental: ~16
// cycles each for one wave).  A wave keeps issuing while its MFMA runs, so an
// MFMA followed by one exponential costs ~20 cycles instead of 16 + 16; the
// segments pair them one to one (the whole step's math: ~1,150 cycles
// instead of ~1,315 with the compiler's own interleave).

// S^T of one step against column tile c: s[t] = K(tile t) . Q(c)^T.
template <int D, class QS>
__device__ __forceinline__ void tile_scores(f32x4 (&s)[2], const KVPair<D>& kv, const QS& qop,
                                            int c) {
  s[0] = f32x4{0.f, 0.f, 0.f, 0.f};
  s[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < Geo<D>::KS; ++ks) {
    const f16x8 qk = qop(c, ks);
    s[0] = mfma16x16x32(kv.k[0][ks], qk, s[0]);
    s[1] = mfma16x16x32(kv.k[1][ks], qk, s[1]);
  }
}

// Scores of keys at or past each lane's column limit (lim(c): the limit of
// the lane's column in column tile c) become -inf.
template <int NCT, class Lim>
__device__ __forceinline__ void mask_scores(f32x4 (&s)[NCT][2], int key0a, int key0b, const Lim& lim,
                                            int grp) {
  const int kba = key0a + 4 * grp;
  const int kbb = key0b + 4 * grp;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int l = lim(c);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[c][0][r] = kba + r < l ? s[c][0][r] : kNegInf;
      s[c][1][r] = kbb + r < l ? s[c][1][r] : kNegInf;
    }
  }
}

// Move the reference max of the column tiles when any lane's raw maximum
// passed its column's threshold (rare; see kRescaleSlack), rescaling the
// state.  Every column tile is updated then: its new max is at least the old
// one, so the rescale factor is at most 1 and o = acc / l is unchanged.
template <int D, int NCT>
__device__ __forceinline__ void update_max(SoftmaxAcc<D, NCT>& st, const f32x4 (&s)[NCT][2],
                                           float scale_log2) {
  float xb[NCT];
  bool need = false;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    xb[c] = fmaxf(fmaxf(fmaxf(s[c][0][0], s[c][0][1]), fmaxf(s[c][0][2], s[c][0][3])),
                  fmaxf(fmaxf(s[c][1][0], s[c][1][1]), fmaxf(s[c][1][2], s[c][1][3])));
    // (scaled against m, not a stored threshold: a register a column tile less)
    need |= __builtin_fmaf(xb[c], scale_log2, -st.m[c]) > kRescaleSlack;
  }
  if (__any(need)) {
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      const float m_new = fmaxf(st.m[c], col_max4(xb[c]) * scale_log2);
      const float alpha = fast_exp2(st.m[c] - m_new);  // 0 for an empty state
      st.m[c] = m_new;
      st.lsum[c][0] *= alpha;
      st.lpart[c] *= alpha;
#pragma unroll
      for (int nt = 0; nt < Geo<D>::NT; ++nt) st.acc[c][nt] *= alpha;
    }
  }
}

// The P.V operands of a step: va[nt] holds, for the lane's output dim of
// d-tile nt, the 8 keys key(grp, e) (a transpose of the loaded V rows).
template <int D>
__device__ __forceinline__ void v_operands(f16x8 (&va)[Geo<D>::NT], const KVPair<D>& kv) {
#pragma unroll
  for (int nt = 0; nt < Geo<D>::NT; ++nt)
#pragma unroll
    for (int e = 0; e < 8; ++e) va[nt][e] = kv.v[e][nt];
}

// One segment of a pipelined step: for column tile c (c < NCT) its
// exponentials and the S MFMAs of its next step's scores, and for tile c - 1
// (c > 0) its P.V MFMAs.  The NT S MFMAs go first, then the NT P.V MFMAs,
// and exponential r of tile c follows MFMA r * 2 * NT / 8, so each MFMA runs
// while the wave issues one exponential (D = 64; every second MFMA for
// D = 128).  The scheduling barriers keep the compiler from regrouping them
// (its own interleave puts the eight exponentials of a tile back to back).
// With the S MFMAs first, the Q^T operands q are free after them:
// next_q(q) then reads the next column tile's into the same registers, a
// segment's worth of P.V MFMAs ahead of their use (reading them at the
// segment's start stalled each segment on the LDS round trip).
// x: 2^x arguments of tile c (s * scale - m); e: the exponentials.
template <int D, int NCT, class NextQ>
__device__ __forceinline__ void step_segment(SoftmaxAcc<D, NCT>& st, int c, const f16x8& pprev,
                                             const f16x8 (&va)[Geo<D>::NT], const KVPair<D>& kv,
                                             f16x8 (&q)[Geo<D>::KS], f32x4 (&s1)[2],
                                             const float (&x)[8], float (&e)[8], NextQ next_q) {
  constexpr int NT = Geo<D>::NT;
  constexpr int NM = 2 * NT;  // 2 * KS = NT S MFMAs, then NT P.V MFMAs
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    if (i < NT) {
      if (c < NCT) {
        // S(t = i % 2, k-step i / 2): a tile's k-steps are 2 MFMAs apart
        const int t = i % 2, ks = i / 2;
        s1[t] = mfma16x16x32(kv.k[t][ks], q[ks], ks == 0 ? zero : s1[t]);
      }
    } else if (c > 0) {
      st.acc[c - 1][i - NT] = mfma16x16x32(va[i - NT], pprev, st.acc[c - 1][i - NT]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (c < NCT && (i * 8) % NM == 0) e[i * 8 / NM] = fast_exp2(x[i * 8 / NM]);
    if (c < NCT && i == NT + 1) next_q(q);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The lane's part of column tile c's row sums += its 8 fp16 P values
// (v_dot2_f32_f16 against (1, 1): exact products, fp32 sums; one register a
// column tile instead of an MFMA output's four).
__device__ __forceinline__ void add_row_sums(float& lpart, const f16x8& p) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 one2 = {(f16)1.f, (f16)1.f};
  float l = lpart;
#pragma unroll
  for (int i = 0; i < 4; ++i) l = __builtin_amdgcn_fdot2(h2{p[2 * i], p[2 * i + 1]}, one2, l, false);
  lpart = l;
}

// stream_tiles with steps overlapped as described above.  Step t's V rows
// are loaded at the start of step t-1 and its K tiles at the start of step
// t-2, so K (needed mid-step, for the S MFMAs one step ahead) has one and a
// half steps of lead and V one.
//
// Loads go through one descriptor per pool (the pool is under 4 GiB: the
// caller checks) with the tile's byte offset as the scalar offset: a step
// costs two v_readlane and no per-tile descriptor (a per-tile descriptor is
// about 17 scalar instructions, which a lone wave per SIMD pays in issue
// slots).  Rows past key_end are then real pool memory: their scores are
// masked like any key past a column's limit, and their V rows are zeroed in
// registers on the steps that hold them (pool memory past a sequence's end
// may hold anything).  Past the last step the loads go through descriptors
// of no records (zeros, no memory access), so every step issues the same
// loads and each wait covers exactly the step it is for.
template <int D, int NCT, class QS, class Lim, class Prologue>
__device__ __forceinline__ void stream_tiles_pipelined(SoftmaxAcc<D, NCT>& st, const QS& qop,
                                                       const Lim& lim, int t_begin,
                                                       int t_end, int key_end,
                                                       const PagedSrc& src, float scale_log2,
                                                       int r16, int grp, Prologue prologue) {
  constexpr int NT = Geo<D>::NT;
  t_begin = uniform(t_begin);
  t_end = uniform(t_end);
  key_end = uniform(key_end);
  if (t_begin >= t_end) {
    prologue();
    return;
  }
  int mask_from = kNoKey;
#pragma unroll
  for (int c = 0; c < NCT; ++c) mask_from = min(mask_from, lim(c));
  for (int off = 1; off < kWave; off <<= 1) mask_from = min(mask_from, __shfl_xor(mask_from, off, kWave));
  mask_from = uniform(mask_from);
  const int lane = threadIdx.x & (kWave - 1);
  const TileLaneOffsets<D> lanes(r16, grp);
  const PoolTiles<D> pool(src, t_end, lane);
  const __amdgpu_buffer_rsrc_t k_none = coherent_rsrc(src.k_pool, 0);
  const __amdgpu_buffer_rsrc_t v_none = coherent_rsrc(src.v_pool, 0);
  int page = pool.lane_page(t_begin);
  prologue();
  for (int c0 = t_begin; c0 < t_end; c0 += kWave) {
    if (c0 != t_begin) page = pool.lane_page(c0);
    const PoolChunk ch(pool, c0, page);
    const int n_pairs = ch.n_pairs;
    // the first steps that need masking and V-row zeroing
    const int j_mask = ch.first_step_past(mask_from);
    const int j_tail = ch.first_step_past(key_end);
    KVPair<D> ring[3];  // K in slot t % 3, V in slot t % 2
    // (the lane offsets pass through an empty asm at each use, so the
    // compiler cannot hoist "offset + constant" out of the loop into extra
    // registers; the constants then go into the loads' immediate offsets)
    // (past the last step the loads go through descriptors of no records:
    // zeros, no memory access)
    auto issue_k = [&](int slot, int j) {
      uint32_t o[2];
      ch.offsets(j, o[0], o[1]);
      uint32_t ko = lanes.k;
      asm volatile("" : "+v"(ko));
      const __amdgpu_buffer_rsrc_t kd = j < n_pairs ? pool.kd : k_none;
#pragma unroll
      for (int n = 0; n < 2 * Geo<D>::KS; ++n) pool_load_k<D>(ring[slot], kd, o, ko, n);
    };
    auto issue_v = [&](int slot, int j) {
      uint32_t o[2];
      ch.offsets(j, o[0], o[1]);
      uint32_t vo = lanes.v;
      asm volatile("" : "+v"(vo));
      const __amdgpu_buffer_rsrc_t vd = j < n_pairs ? pool.vd : v_none;
#pragma unroll
      for (int n = 0; n < 8; ++n) pool_load_v<D>(ring[slot], vd, o, vo, n);
    };
    auto step_keys = [&](int j, int& ka, int& kb) { ch.step_keys(j, ka, kb); };
    issue_k(0, 0);
    issue_v(0, 0);
    issue_k(1, 1);
    f32x4 s[NCT][2];
#pragma unroll
    for (int c = 0; c < NCT; ++c) tile_scores<D>(s[c], ring[0], qop, c);
    if (j_mask == 0) {
      int ka, kb;
      step_keys(0, ka, kb);
      mask_scores<NCT>(s, ka, kb, lim, grp);
    }
    update_max<D, NCT>(st, s, scale_log2);
    // Q^T operands of the next segment's column tile (carried across steps)
    f16x8 q[Geo<D>::KS];
#pragma unroll
    for (int ks = 0; ks < Geo<D>::KS; ++ks) q[ks] = qop(0, ks);
    for (int j0 = 0; j0 < n_pairs; j0 += 6) {
#pragma unroll
      for (int u = 0; u < 6; ++u) {
        const int j = j0 + u;
        if (j < n_pairs) {
          if (j >= j_tail) {
            int ka, kb;
            step_keys(j, ka, kb);
            zero_tail_rows<D>(ring[u % 2], ka, kb, key_end, grp);
          }
          f16x8 va[NT];
          v_operands<D>(va, ring[u % 2]);
          issue_v((u + 1) % 2, j + 1);
          issue_k((u + 2) % 3, j + 2);
          // Segment c: the exponentials of column tile c, the P.V MFMAs of
          // tile c - 1 and the S MFMAs of tile c for the next step.
          // Scheduling barriers between segments keep each step's scores
          // consumed as the next step's are produced (registers).
          f32x4 s1[NCT][2];
          f16x8 pprev;
#pragma unroll
          for (int c = 0; c <= NCT; ++c) {
            __builtin_amdgcn_sched_barrier(0);
            float x[8], e[8];
            if (c < NCT) {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                x[r] = __builtin_fmaf(s[c][0][r], scale_log2, -st.m[c]);
                x[4 + r] = __builtin_fmaf(s[c][1][r], scale_log2, -st.m[c]);
              }
            }
            // (tile c + 1's Q^T operands, or tile 0's for the next step)
            auto next_q = [&](f16x8 (&qq)[Geo<D>::KS]) {
#pragma unroll
              for (int ks = 0; ks < Geo<D>::KS; ++ks) qq[ks] = qop((c + 1) % NCT, ks);
            };
            step_segment<D, NCT>(st, c, pprev, va, ring[(u + 1) % 3], q, s1[c < NCT ? c : 0], x, e,
                                 next_q);
            if (c > 0) add_row_sums(st.lpart[c - 1], pprev);
            if (c < NCT) {
#pragma unroll
              for (int r = 0; r < 8; ++r) pprev[r] = (f16)e[r];
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          if (j + 1 < n_pairs) {
            if (j + 1 >= j_mask) {
              int ka, kb;
              step_keys(j + 1, ka, kb);
              mask_scores<NCT>(s1, ka, kb, lim, grp);
            }
            update_max<D, NCT>(st, s1, scale_log2);
          }
#pragma unroll
          for (int c = 0; c < NCT; ++c) {
            s[c][0] = s1[c][0];
            s[c][1] = s1[c][1];
          }
        }
      }
    }
  }
}

}  // namespace cie
