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

template <int D>
__device__ __forceinline__ void load_pair(KVPair<D>& kv, const f16* __restrict__ kpool,
                                          const f16* __restrict__ vpool, TileLoc t0,
                                          TileLoc t1, bool two, int r16, int grp) {
  constexpr int KS = Geo<D>::KS;
  constexpr int NT = Geo<D>::NT;
  typedef typename HVec<NT>::type vrow_t;
  const f16* k0 = kpool + t0.base + r16 * D + 8 * grp;
  const f16* v0 = vpool + t0.base + (4 * grp) * D + NT * r16;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kv.k[0][ks] = *reinterpret_cast<const f16x8*>(k0 + 32 * ks);
#pragma unroll
  for (int e = 0; e < 4; ++e) kv.v[e] = *reinterpret_cast<const vrow_t*>(v0 + e * D);
  if (two) {
    const f16* k1 = kpool + t1.base + r16 * D + 8 * grp;
    const f16* v1 = vpool + t1.base + (4 * grp) * D + NT * r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kv.k[1][ks] = *reinterpret_cast<const f16x8*>(k1 + 32 * ks);
#pragma unroll
    for (int e = 0; e < 4; ++e) kv.v[4 + e] = *reinterpret_cast<const vrow_t*>(v1 + e * D);
  } else {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kv.k[1][ks] = f16x8{};
#pragma unroll
    for (int e = 0; e < 4; ++e) kv.v[4 + e] = vrow_t{};
  }
}

// Zero the V rows at keys >= key_end (the masked loads of the reference read
// 0 there; pool memory past a sequence's end may hold anything).  key0a /
// key0b: first key of the pair's two tiles.
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

// Online-softmax state for NCT 16-wide column tiles held by one wave.
template <int D, int NCT>
struct SoftmaxAcc {
  float m[NCT];  // running max (log2 domain), identical across a column's 4 lanes
  float l[NCT];  // lane-partial running sum (reduced over the 4 lanes at the end)
  f32x4 acc[NCT][Geo<D>::NT];

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      m[c] = kNegInf;
      l[c] = 0.f;
#pragma unroll
      for (int nt = 0; nt < Geo<D>::NT; ++nt) acc[c][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
};

// One 32-key step for NCT column tiles.  key0a / key0b = absolute index of the
// first key of the pair's two tiles (the tiles need not be adjacent; an absent
// second tile passes kNoKey).  A column attends key j iff j < lim[c] (per
// lane: causal / length limit of the lane's column); mask_from (wave-uniform)
// is the smallest limit of any column, so steps whose keys all lie below it
// skip the masking.
//
// The column tiles go in batches of up to kAttendBatch; a batch runs in
// phases — its Q.K^T MFMAs, its columns' softmax updates, one (rare) rescale,
// its P.V MFMAs — with no branch inside a phase, so one wave overlaps a column
// tile's softmax with the MFMAs of the others.  VALU per column tile: the max
// runs on raw scores (the scale is positive), exp2 takes fma(s, scale, -m),
// and the accumulator rescale is skipped when no column's max moved
// (alpha == 1 exactly).
#ifndef CIE_ATTEND_BATCH
#define CIE_ATTEND_BATCH 4
#endif
constexpr int kAttendBatch = CIE_ATTEND_BATCH;

template <int D, int NCT, bool MASK>
__device__ __forceinline__ void attend_pair_body(SoftmaxAcc<D, NCT>& st, const KVPair<D>& kv,
                                                 const f16x8 (&qop)[NCT][Geo<D>::KS], int key0a,
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
          s[i][0] = mfma16x16x32(kv.k[0][ks], qop[c0 + i][ks], s[i][0]);
          s[i][1] = mfma16x16x32(kv.k[1][ks], qop[c0 + i][ks], s[i][1]);
        }
      }
    }
    f16x8 pop[SB];
    float alpha[SB];
    bool moved = false;
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (c0 + i < NCT) {
        const int c = c0 + i;
        float sc[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[r] = s[i][0][r];
          sc[4 + r] = s[i][1][r];
        }
        if constexpr (MASK) {
          const int kba = key0a + 4 * grp;
          const int kbb = key0b + 4 * grp;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sc[r] = kba + r < lim[c] ? sc[r] : kNegInf;
            sc[4 + r] = kbb + r < lim[c] ? sc[4 + r] : kNegInf;
          }
        }
        float mb = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                         fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
        mb = col_max4(mb) * scale_log2;
        const float m_new = fmaxf(st.m[c], mb);
        // A column with every key masked so far keeps m = -inf, l = 0,
        // acc = 0; m_use keeps exp2 away from (-inf) - (-inf).
        const float m_use = (m_new == kNegInf) ? 0.f : m_new;
        alpha[i] = fast_exp2(st.m[c] - m_use);
        moved |= alpha[i] != 1.f;
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = fast_exp2(__builtin_fmaf(sc[e], scale_log2, -m_use));
          ps += pe;
          pop[i][e] = (f16)pe;
        }
        st.l[c] = __builtin_fmaf(st.l[c], alpha[i], ps);
        st.m[c] = m_new;
      }
    }
    if (__any(moved)) {
#pragma unroll
      for (int i = 0; i < SB; ++i)
        if (c0 + i < NCT)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) st.acc[c0 + i][nt] *= alpha[i];
    }
#pragma unroll
    for (int i = 0; i < SB; ++i)
      if (c0 + i < NCT)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          st.acc[c0 + i][nt] = mfma16x16x32(va[nt], pop[i], st.acc[c0 + i][nt]);
  }
}

template <int D, int NCT>
__device__ __forceinline__ void attend_pair(SoftmaxAcc<D, NCT>& st, const KVPair<D>& kv,
                                            const f16x8 (&qop)[NCT][Geo<D>::KS], int key0a,
                                            int key0b, const int (&lim)[NCT], int mask_from,
                                            float scale_log2, int grp) {
  if (max(key0a, key0b) + 16 > mask_from)  // uniform
    attend_pair_body<D, NCT, true>(st, kv, qop, key0a, key0b, lim, scale_log2, grp);
  else
    attend_pair_body<D, NCT, false>(st, kv, qop, key0a, key0b, lim, scale_log2, grp);
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
};

// Stream key tiles [t_begin, t_end) of one wave through attend_pair, two
// tiles per step.  The page ids of up to 64 tiles are gathered first, one per
// lane, so a step's K/V loads depend on no other load; a ring of PF + 1
// register-staged steps keeps PF steps of loads in flight ahead of the math.
// key_end = number of keys that exist (rows at or past it are zeroed).
template <int D, int NCT, int PF>
__device__ __forceinline__ void stream_tiles(SoftmaxAcc<D, NCT>& st,
                                             const f16x8 (&qop)[NCT][Geo<D>::KS],
                                             const int (&lim)[NCT], int t_begin, int t_end,
                                             int key_end, const PagedSrc& src, float scale_log2,
                                             int r16, int grp) {
  if (t_begin >= t_end) return;
  int mask_from = kNoKey;
#pragma unroll
  for (int c = 0; c < NCT; ++c) mask_from = min(mask_from, lim[c]);
  // smallest limit over the wave's columns (wave-uniform)
  for (int off = 1; off < kWave; off <<= 1) mask_from = min(mask_from, __shfl_xor(mask_from, off, kWave));
  const int lane = threadIdx.x & (kWave - 1);
  const int tpp = src.page_size >> 4;  // 16-key tiles per page
  for (int c0 = t_begin; c0 < t_end; c0 += kWave) {
    const int n_chunk = min(kWave, t_end - c0);
    int page = 0;
    if (lane < n_chunk) {
      int64_t pg = src.bt_row[(c0 + lane) / tpp];
      if (pg < 0 || pg >= src.n_pages) {
        set_err(src.err, CIE_ERRBIT_PAGE);
        pg = 0;
      }
      page = (int)pg;
    }
    const int n_pairs = (n_chunk + 1) >> 1;
    KVPair<D> ring[PF + 1];
    int keya[PF + 1], keyb[PF + 1];
    auto issue = [&](int slot, int j) {
      const int ka = 2 * j;  // chunk-local index of the step's first tile
      const bool two = ka + 1 < n_chunk;
      const int ta = c0 + ka;
      const int pa = __builtin_amdgcn_readlane(page, ka);
      const int pb = two ? __builtin_amdgcn_readlane(page, ka + 1) : pa;
      const TileLoc l0{(int64_t)pa * src.page_stride + src.head_off + (int64_t)((ta % tpp) * 16) * D};
      const TileLoc l1{(int64_t)pb * src.page_stride + src.head_off +
                       (int64_t)(((ta + 1) % tpp) * 16) * D};
      keya[slot] = ta * 16;
      keyb[slot] = two ? ta * 16 + 16 : kNoKey;
      load_pair<D>(ring[slot], src.k_pool, src.v_pool, l0, l1, two, r16, grp);
    };
#pragma unroll
    for (int j = 0; j < PF; ++j)
      if (j < n_pairs) issue(j, j);
    for (int j0 = 0; j0 < n_pairs; j0 += PF + 1) {
#pragma unroll
      for (int u = 0; u <= PF; ++u) {
        const int j = j0 + u;
        if (j < n_pairs) {
          if (j + PF < n_pairs) issue((u + PF) % (PF + 1), j + PF);
          const int ka = keya[u], kb = keyb[u];
          if ((kb == kNoKey ? ka : kb) + 16 > key_end) zero_tail_rows<D>(ring[u], ka, kb, key_end, grp);
          attend_pair<D, NCT>(st, ring[u], qop, ka, kb, lim, mask_from, scale_log2, grp);
        }
      }
    }
  }
}

}  // namespace cie
