// KV append into the paged pool: the new tokens' K/V rows are scattered into
// (page, in-page offset) slots of the (n_pages, H_kv, page_size, D) pools.
//
// One launch covers K and V of every (token, kv head).  A lane moves one
// VEC-wide chunk of one row for both K and V, lanes of a row are adjacent, so
// the reads of k_new/v_new and the 2*D-byte row writes into the pool are
// coalesced.  The copy is a pure fp16 move: bit-exact by construction.
//
// Decode mode follows KVStorage.decode_update (kv_cache/storage.py:87-122):
//   pos = lens[slot]; page = block_table[slot, pos // page_size];
//   off = pos % page_size.
// Token mode follows KVStorage.mixed_update (kv_cache/storage.py:62-85):
//   page = pages[t]; off = offsets[t].
#include "cie_common.h"

namespace cie {

struct AppendParams {
  f16* k_pool;
  f16* v_pool;
  const f16* k_new;
  const f16* v_new;
  int64_t k_tok_stride, k_head_stride, v_tok_stride, v_head_stride;
  // decode mode
  const int64_t* slot_ids;
  const int64_t* lens;
  const int64_t* block_table;
  int64_t bt_stride;
  int64_t bt_width;
  int64_t n_slots;
  // token mode
  const int64_t* pages;
  const int64_t* offsets;
  // common
  int64_t n_rows;  // B (decode) or T (tokens)
  int64_t n_pages;
  int64_t pool_page_stride, pool_head_stride;
  int32_t H_kv, page_size, D;
  int32_t* err;
};

template <int VEC, bool kDecode>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
  typedef f16 vec_t __attribute__((ext_vector_type(VEC)));
  const int chunks = p.D / VEC;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = p.n_rows * p.H_kv * chunks;
  if (gid >= total) return;
  const int c = (int)(gid % chunks);
  const int h = (int)((gid / chunks) % p.H_kv);
  const int64_t row = gid / ((int64_t)chunks * p.H_kv);

  // Every load that does not depend on another goes out first: the new rows
  // (always in bounds) and the row's index (slot id, or page and offset), so
  // the kernel's memory round trips are only the ones the index chain forces
  // (decode: slot -> lens[slot] -> block_table[slot, pos / page_size]; token
  // mode: none after the first).  The checks come after the loads: an error
  // store between two loads would make the second wait for the first.
  const vec_t kv = *reinterpret_cast<const vec_t*>(p.k_new + row * p.k_tok_stride +
                                                   h * p.k_head_stride + c * VEC);
  const vec_t vv = *reinterpret_cast<const vec_t*>(p.v_new + row * p.v_tok_stride +
                                                   h * p.v_head_stride + c * VEC);
  int64_t page, off;
  if constexpr (kDecode) {
    const int64_t slot = p.slot_ids[row];
    const bool slot_ok = slot >= 0 && slot < p.n_slots;
    const int64_t pos = p.lens[slot_ok ? slot : 0];
    const bool pos_ok = pos >= 0 && pos < p.bt_width * p.page_size;
    page = p.block_table[(slot_ok ? slot : 0) * p.bt_stride + (pos_ok ? pos / p.page_size : 0)];
    off = pos % p.page_size;
    if (!slot_ok) {
      set_err(p.err, CIE_ERRBIT_PAGE);
      return;
    }
    if (!pos_ok) {
      set_err(p.err, CIE_ERRBIT_LEN);
      return;
    }
  } else {
    page = p.pages[row];
    off = p.offsets[row];
    if (off < 0 || off >= p.page_size) {
      set_err(p.err, CIE_ERRBIT_OFFSET);
      return;
    }
  }
  if (page < 0 || page >= p.n_pages) {
    set_err(p.err, CIE_ERRBIT_PAGE);
    return;
  }
  const int64_t dst = page * p.pool_page_stride + h * p.pool_head_stride + off * p.D + (int64_t)c * VEC;
  *reinterpret_cast<vec_t*>(p.k_pool + dst) = kv;
  *reinterpret_cast<vec_t*>(p.v_pool + dst) = vv;
}

// Token mode from the fused QKV projection, with RoPE: row t of qkv holds
// q (H_q heads), k (H_kv) and v (H_kv), D each.  A lane takes dims [8c, 8c+8)
// and their rotate_half partners [8c + D/2, ...) of one (token, head): q heads
// are rotated into q_out (T, H_q, D); kv heads have K rotated and V copied
// into (pages[t], head, offsets[t]) of the pools.  This is the QKV split,
// apply_rotary_pos_emb and KVStorage.mixed_update of TritonQwen2Attention's
// mixed branch (attn/core.py:181-198, 226-229) in one launch.
struct QkvRopeParams {
  f16* q_out;
  f16* k_pool;
  f16* v_pool;
  const f16* qkv;
  const f16* cos;
  const f16* sin;
  const int64_t* pages;
  const int64_t* offsets;
  int64_t qkv_stride, cs_stride;
  int64_t T, n_pages, pool_page_stride, pool_head_stride;
  int32_t H_q, H_kv, page_size, D;
  int32_t* err;
};

__global__ __launch_bounds__(256) void qkv_rope_append_kernel(QkvRopeParams p) {
  const int halves = p.D / 16;  // lanes per (token, head)
  const int heads = p.H_q + p.H_kv;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.T * heads * halves) return;
  const int c = (int)(gid % halves);
  const int h = (int)((gid / halves) % heads);
  const int64_t t = gid / ((int64_t)halves * heads);
  const int half = p.D / 2;
  const int d0 = 8 * c;

  // All loads first (one memory round trip): the token's rotary rows, its
  // q / k / v dims, and for kv heads the page and in-page offset.
  const bool kv_head = h >= p.H_q;
  const f16* crow = p.cos + t * p.cs_stride;
  const f16* srow = p.sin + t * p.cs_stride;
  const f16x8 c_lo = *reinterpret_cast<const f16x8*>(crow + d0);
  const f16x8 c_hi = *reinterpret_cast<const f16x8*>(crow + d0 + half);
  const f16x8 s_lo = *reinterpret_cast<const f16x8*>(srow + d0);
  const f16x8 s_hi = *reinterpret_cast<const f16x8*>(srow + d0 + half);
  const f16* x = p.qkv + t * p.qkv_stride + (int64_t)h * p.D;
  f16x8 lo = *reinterpret_cast<const f16x8*>(x + d0);
  f16x8 hi = *reinterpret_cast<const f16x8*>(x + d0 + half);
  f16x8 v_lo = {}, v_hi = {};
  int64_t page = 0, off = 0;
  if (kv_head) {
    const f16* v = x + (int64_t)p.H_kv * p.D;  // v block: H_kv heads after k
    v_lo = *reinterpret_cast<const f16x8*>(v + d0);
    v_hi = *reinterpret_cast<const f16x8*>(v + d0 + half);
    page = p.pages[t];
    off = p.offsets[t];
  }
  rope8(lo, hi, c_lo, c_hi, s_lo, s_hi);

  if (!kv_head) {
    f16* dst = p.q_out + (t * p.H_q + h) * p.D;
    *reinterpret_cast<f16x8*>(dst + d0) = lo;
    *reinterpret_cast<f16x8*>(dst + d0 + half) = hi;
    return;
  }
  if (off < 0 || off >= p.page_size) {
    set_err(p.err, CIE_ERRBIT_OFFSET);
    return;
  }
  if (page < 0 || page >= p.n_pages) {
    set_err(p.err, CIE_ERRBIT_PAGE);
    return;
  }
  const int hk = h - p.H_q;
  const int64_t row = page * p.pool_page_stride + hk * p.pool_head_stride + off * p.D;
  *reinterpret_cast<f16x8*>(p.k_pool + row + d0) = lo;
  *reinterpret_cast<f16x8*>(p.k_pool + row + d0 + half) = hi;
  *reinterpret_cast<f16x8*>(p.v_pool + row + d0) = v_lo;
  *reinterpret_cast<f16x8*>(p.v_pool + row + d0 + half) = v_hi;
}

static bool aligned16(const void* ptr) {
  return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0;
}

template <bool kDecode>
static int launch_append(const AppendParams& p, hipStream_t stream) {
  if (p.n_rows == 0) return CIE_OK;
  const bool vec8 = (p.D % 8 == 0) && aligned16(p.k_pool) && aligned16(p.v_pool) &&
                    aligned16(p.k_new) && aligned16(p.v_new) &&
                    p.k_tok_stride % 8 == 0 && p.k_head_stride % 8 == 0 &&
                    p.v_tok_stride % 8 == 0 && p.v_head_stride % 8 == 0 &&
                    p.pool_page_stride % 8 == 0 && p.pool_head_stride % 8 == 0;
  const int vec = vec8 ? 8 : 1;
  const int64_t total = p.n_rows * p.H_kv * (p.D / vec);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return CIE_EUNSUPPORTED;
  if (vec8)
    hipLaunchKernelGGL((kv_append_kernel<8, kDecode>), dim3((unsigned)blocks),
                       dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((kv_append_kernel<1, kDecode>), dim3((unsigned)blocks),
                       dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

}  // namespace cie

using namespace cie;

extern "C" int cie_kv_append_decode(
    void* k_pool, void* v_pool, const void* k_new, const void* v_new,
    int64_t k_tok_stride, int64_t k_head_stride, int64_t v_tok_stride,
    int64_t v_head_stride, const int64_t* slot_ids, const int64_t* lens,
    const int64_t* block_table, int64_t B, int64_t H_kv, int64_t page_size,
    int64_t D, int64_t n_pages, int64_t pool_page_stride,
    int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
    int64_t n_slots, int32_t* err, void* stream) {
  if (B < 0 || H_kv <= 0 || page_size <= 0 || D <= 0 || n_pages <= 0 ||
      bt_width <= 0 || bt_stride < bt_width || n_slots <= 0)
    return CIE_EINVAL;
  if (B > 0 && (!k_pool || !v_pool || !k_new || !v_new || !slot_ids || !lens ||
                !block_table))
    return CIE_EINVAL;
  if (H_kv > 0x7fffffff || page_size > 0x7fffffff || D > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  AppendParams p{};
  p.k_pool = static_cast<f16*>(k_pool);
  p.v_pool = static_cast<f16*>(v_pool);
  p.k_new = static_cast<const f16*>(k_new);
  p.v_new = static_cast<const f16*>(v_new);
  p.k_tok_stride = k_tok_stride;
  p.k_head_stride = k_head_stride;
  p.v_tok_stride = v_tok_stride;
  p.v_head_stride = v_head_stride;
  p.slot_ids = slot_ids;
  p.lens = lens;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.bt_width = bt_width;
  p.n_slots = n_slots;
  p.n_rows = B;
  p.n_pages = n_pages;
  p.pool_page_stride = pool_page_stride;
  p.pool_head_stride = pool_head_stride;
  p.H_kv = (int32_t)H_kv;
  p.page_size = (int32_t)page_size;
  p.D = (int32_t)D;
  p.err = err;
  return launch_append<true>(p, static_cast<hipStream_t>(stream));
}

extern "C" int cie_kv_append_tokens(
    void* k_pool, void* v_pool, const void* k_new, const void* v_new,
    int64_t k_tok_stride, int64_t k_head_stride, int64_t v_tok_stride,
    int64_t v_head_stride, const int64_t* pages, const int64_t* offsets,
    int64_t T, int64_t H_kv, int64_t page_size, int64_t D, int64_t n_pages,
    int64_t pool_page_stride, int64_t pool_head_stride, int32_t* err,
    void* stream) {
  if (T < 0 || H_kv <= 0 || page_size <= 0 || D <= 0 || n_pages <= 0)
    return CIE_EINVAL;
  if (T > 0 && (!k_pool || !v_pool || !k_new || !v_new || !pages || !offsets))
    return CIE_EINVAL;
  if (H_kv > 0x7fffffff || page_size > 0x7fffffff || D > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  AppendParams p{};
  p.k_pool = static_cast<f16*>(k_pool);
  p.v_pool = static_cast<f16*>(v_pool);
  p.k_new = static_cast<const f16*>(k_new);
  p.v_new = static_cast<const f16*>(v_new);
  p.k_tok_stride = k_tok_stride;
  p.k_head_stride = k_head_stride;
  p.v_tok_stride = v_tok_stride;
  p.v_head_stride = v_head_stride;
  p.pages = pages;
  p.offsets = offsets;
  p.n_rows = T;
  p.n_pages = n_pages;
  p.pool_page_stride = pool_page_stride;
  p.pool_head_stride = pool_head_stride;
  p.H_kv = (int32_t)H_kv;
  p.page_size = (int32_t)page_size;
  p.D = (int32_t)D;
  p.err = err;
  return launch_append<false>(p, static_cast<hipStream_t>(stream));
}

extern "C" int cie_kv_append_tokens_qkv_rope(
    void* q_out, void* k_pool, void* v_pool, const void* qkv, int64_t qkv_row_stride,
    const void* cos, const void* sin, int64_t cs_row_stride, const int64_t* pages,
    const int64_t* offsets, int64_t T, int64_t H_q, int64_t H_kv, int64_t page_size, int64_t D,
    int64_t n_pages, int64_t pool_page_stride, int64_t pool_head_stride, int32_t* err,
    void* stream) {
  if (T < 0 || H_q <= 0 || H_kv <= 0 || page_size <= 0 || D <= 0 || n_pages <= 0)
    return CIE_EINVAL;
  if (D % 16 != 0 || H_q + H_kv > 0x7fffffff || page_size > 0x7fffffff || D > 0x7fffffff)
    return CIE_EUNSUPPORTED;
  if (T == 0) return CIE_OK;
  if (!q_out || !k_pool || !v_pool || !qkv || !cos || !sin || !pages || !offsets)
    return CIE_EINVAL;
  if (!aligned16(q_out) || !aligned16(k_pool) || !aligned16(v_pool) || !aligned16(qkv) ||
      !aligned16(cos) || !aligned16(sin) || qkv_row_stride % 8 != 0 || cs_row_stride % 8 != 0 ||
      pool_page_stride % 8 != 0 || pool_head_stride % 8 != 0 ||
      qkv_row_stride < (H_q + 2 * H_kv) * D || cs_row_stride < D)
    return CIE_EINVAL;
  QkvRopeParams p{};
  p.q_out = static_cast<f16*>(q_out);
  p.k_pool = static_cast<f16*>(k_pool);
  p.v_pool = static_cast<f16*>(v_pool);
  p.qkv = static_cast<const f16*>(qkv);
  p.cos = static_cast<const f16*>(cos);
  p.sin = static_cast<const f16*>(sin);
  p.pages = pages;
  p.offsets = offsets;
  p.qkv_stride = qkv_row_stride;
  p.cs_stride = cs_row_stride;
  p.T = T;
  p.n_pages = n_pages;
  p.pool_page_stride = pool_page_stride;
  p.pool_head_stride = pool_head_stride;
  p.H_q = (int32_t)H_q;
  p.H_kv = (int32_t)H_kv;
  p.page_size = (int32_t)page_size;
  p.D = (int32_t)D;
  p.err = err;
  const int64_t total = T * (H_q + H_kv) * (D / 16);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return CIE_EUNSUPPORTED;
  hipLaunchKernelGGL(qkv_rope_append_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p);
  return (int)hipGetLastError();
}
