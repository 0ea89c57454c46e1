/*
 * cie_paged_attention.h — C ABI of the MI355X (gfx950) paged-KV GQA attention
 * hot path: KV append, split-KV decode (load + merge) and the varlen mixed
 * (chunked prefill + decode) causal kernel.
 *
 * Conventions shared by every entry point
 * ---------------------------------------
 *  - Every pointer is a device pointer owned by the caller.  Nothing here
 *    allocates, frees or synchronises; kernels are enqueued on `stream`
 *    (a hipStream_t passed as void*; NULL = the null stream), so the calls are
 *    safe under hipGraph stream capture.
 *  - fp16 tensors are IEEE binary16.  Index tensors are int64, the dtype the
 *    reference uses for lens / slot ids / block tables / cu_seqlens.
 *  - KV pool layout is the reference's (n_pages, H_kv, page_size, D) with the
 *    last two dims dense (stride(3) == 1, stride(2) == D); the page and head
 *    strides are passed explicitly (in elements).
 *  - The block table is (n_slots, bt_stride) int64; only the first bt_width
 *    entries of a row are valid logical pages.
 *  - `err` (nullable) is an int32 device word.  Kernels never fault on a bad
 *    index: an out-of-range page id, slot id or length is clamped / skipped and
 *    the matching CIE_ERRBIT_* bit is OR-ed into *err.
 *  - Return value: 0 on success, a negative CIE_E* code for an argument error
 *    detected on the host (nothing is launched), or a positive hipError_t from
 *    the launch.
 */
#ifndef CIE_PAGED_ATTENTION_H
#define CIE_PAGED_ATTENTION_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CIE_OK 0
#define CIE_EINVAL (-1)      /* inconsistent sizes / strides / null pointer      */
#define CIE_EUNSUPPORTED (-2) /* shape outside what the kernels are built for   */
#define CIE_ESCRATCH (-3)     /* problem larger than the static scratch of an
                                 allocation-free entry point                     */

#define CIE_ERRBIT_PAGE 1     /* page id outside [0, n_pages)                    */
#define CIE_ERRBIT_LEN 2      /* length beyond the block-table row capacity      */
#define CIE_ERRBIT_OFFSET 4   /* in-page offset outside [0, page_size)           */
#define CIE_ERRBIT_SPLIT 8    /* a split-arrival counter held a stale value at the
                                 start of the call (see `counters` below)        */
#define CIE_ERRBIT_PLAN 16    /* a planned call whose plan was made for another
                                 batch shape or partials budget (the call wrote
                                 nothing), or a batch with more work items than
                                 its plan holds (cie_mixed_plan)                  */

/* Version of this ABI (bumped on any signature change). */
int cie_abi_version(void);

/* Human-readable name of a CIE_E* / hipError_t status. */
const char* cie_status_string(int status);

/*
 * Decode KV append: for each sequence b, pos = lens[slot_ids[b]],
 *   k_pool[block_table[slot, pos / page_size], h, pos % page_size, :] = k_new[b, h, :]
 * (same for V).  Bit-exact fp16 copy.
 * Replaces KVStorage.decode_update (kv_cache/storage.py:87-122): the torch
 * gather of lens / block_table plus two index_put_ scatters.
 * k_new / v_new are (B, H_kv, D) views with their own token and head strides
 * (elements); the last dim must be dense.
 */
int cie_kv_append_decode(void* k_pool, void* v_pool,
                         const void* k_new, const void* v_new,
                         int64_t k_tok_stride, int64_t k_head_stride,
                         int64_t v_tok_stride, int64_t v_head_stride,
                         const int64_t* slot_ids, const int64_t* lens,
                         const int64_t* block_table,
                         int64_t B, int64_t H_kv, int64_t page_size, int64_t D,
                         int64_t n_pages, int64_t pool_page_stride,
                         int64_t pool_head_stride, int64_t bt_stride,
                         int64_t bt_width, int64_t n_slots,
                         int32_t* err, void* stream);

/*
 * Token-mode (mixed) KV append: for each packed token t < T,
 *   k_pool[pages[t], h, offsets[t], :] = k_new[t, h, :]   (same for V).
 * Replaces KVStorage.mixed_update (kv_cache/storage.py:62-85).
 */
int cie_kv_append_tokens(void* k_pool, void* v_pool,
                         const void* k_new, const void* v_new,
                         int64_t k_tok_stride, int64_t k_head_stride,
                         int64_t v_tok_stride, int64_t v_head_stride,
                         const int64_t* pages, const int64_t* offsets,
                         int64_t T, int64_t H_kv, int64_t page_size, int64_t D,
                         int64_t n_pages, int64_t pool_page_stride,
                         int64_t pool_head_stride, int32_t* err, void* stream);

/*
 * Split-KV paged GQA decode, one query token per sequence:
 *   o[b, h, :] = softmax(q[b, h, :] . K_b^T * D^-0.5) . V_b
 * over the first lens[b] tokens of slot slot_ids[b]'s pages, kv head h / G.
 * lens[b] == 0 gives o = 0.  One kernel launch: the KV splits, and the
 * log-sum-exp merge done by the last workgroup of each (sequence, kv head).
 * Replaces decode_gqa_attention (attn/core.py:13-66), i.e. the Triton
 * decode_gqa_attention_kernel_load (kernels/decode_attention.py:12-179) and
 * decode_attention_kernel_merge (kernels/decode_attention.py:182-272).
 *   q, o       : (B, H_q, D) dense fp16, 16-byte aligned
 *   lens       : (B,) attended lengths (the reference passes lens[slot] + 1)
 *   n_splits   : KV splits per (sequence, kv head) — the reference's
 *                `num_programs`
 *                (1 <= n_splits <= cie_paged_decode_max_splits())
 *   partials   : cie_paged_decode_partials_bytes(B, H_q, D, n_splits) bytes,
 *                16-byte aligned, any contents: the splits' softmax state
 *   counters   : 2 * B * H_kv int32, 16-byte aligned: one arrival word per
 *                (sequence, kv head), then one stale word per (sequence, kv
 *                head).  They must be zero before the call and every
 *                completed call leaves them zero, so one zeroed buffer serves
 *                any number of stream-ordered calls.  Calls that can overlap
 *                in time must not share counters or partials.  A call that
 *                finds an arrival word outside [0, n_splits) raises
 *                CIE_ERRBIT_SPLIT (its o is then not valid); when every split
 *                of a (sequence, kv head) finds it stale, the call also puts
 *                both words back to zero.  A stale value inside [0, n_splits)
 *                cannot be told apart from live arrivals and may survive the
 *                call, so after CIE_ERRBIT_SPLIT the caller zeroes the
 *                counters before the next call.
 *   partials and counters may be NULL when n_splits == 1.
 */
int64_t cie_paged_decode_partials_bytes(int64_t B, int64_t H_q, int64_t D,
                                        int64_t n_splits);
int cie_paged_decode_max_splits(void);
int cie_paged_decode(void* o, const void* q,
                     const void* k_pool, const void* v_pool,
                     const int64_t* lens, const int64_t* slot_ids,
                     const int64_t* block_table,
                     void* partials, int32_t* counters,
                     int64_t B, int64_t H_q, int64_t H_kv, int64_t D,
                     int64_t page_size, int64_t n_pages,
                     int64_t pool_page_stride, int64_t pool_head_stride,
                     int64_t bt_stride, int64_t bt_width, int64_t n_slots,
                     int64_t n_splits, int32_t* err, void* stream);

/*
 * Decode step with the KV append fused in, one launch: for each sequence b,
 * pos = lens[slot_ids[b]] (the pool's prior length per slot, (n_slots,)),
 * the new K/V rows k_new[b] / v_new[b] are written to
 * (block_table[slot, pos / page_size], pos % page_size) bit-exactly, and o is
 * the decode attention over the pos + 1 tokens that then exist.
 * Equivalent to KVStorage.decode_update (kv_cache/storage.py:87-122) followed
 * by gqa_decode_attention with lens[slot] + 1 (attn/core.py:200-215).
 * partials / counters as for cie_paged_decode.
 */
int cie_paged_decode_append(void* o, const void* q, void* k_pool, void* v_pool,
                            const void* k_new, const void* v_new,
                            int64_t k_tok_stride, int64_t k_head_stride,
                            int64_t v_tok_stride, int64_t v_head_stride,
                            const int64_t* lens, const int64_t* slot_ids,
                            const int64_t* block_table, void* partials,
                            int32_t* counters,
                            int64_t B, int64_t H_q, int64_t H_kv, int64_t D,
                            int64_t page_size, int64_t n_pages,
                            int64_t pool_page_stride, int64_t pool_head_stride,
                            int64_t bt_stride, int64_t bt_width,
                            int64_t n_slots, int64_t n_splits, int32_t* err,
                            void* stream);

/*
 * Planned decode.  The slot ids, lengths and block-table rows a decode step
 * reads are the same for every layer of the step (KVStorage advances the
 * lengths after the last layer), so a step can make a plan once and run each
 * layer's decode from it:
 *   cie_paged_decode_plan       once per step: each sequence's attended
 *                               length (append = 1: lens is (n_slots,) prior
 *                               lengths, attended = lens[slot] + 1, as
 *                               cie_paged_decode_append; append = 0: lens is
 *                               (B,) attended lengths, as cie_paged_decode),
 *                               its splits (balanced by length over the
 *                               n_workgroups of the grid) and each workgroup's
 *                               page ids, into `plan`
 *                               (cie_paged_decode_plan_bytes(n_workgroups)
 *                               bytes, 16-byte aligned, any contents).  Index
 *                               errors are reported here (CIE_ERRBIT_*).
 *   cie_paged_decode_planned,   per layer: the same results as
 *   cie_paged_decode_append_planned,   cie_paged_decode / _append / _qkv_rope
 *   cie_paged_decode_qkv_rope_planned  on the plan's sequences, but the
 *                               launch reads one descriptor and its page ids
 *                               instead of the slot id, then the block table
 *                               and the length: one memory round trip less
 *                               before its first K/V loads.
 * The plan must be made with the same append mode, block table and lengths
 * as the layers' calls, and n_workgroups must be the same for all of them.
 * n_workgroups = cie_paged_decode_plan_workgroups(B, H_kv, n_splits):
 * B * H_kv * n_splits, or with n_splits = 0 the library's default (about
 * one workgroup per CU, at least one per (sequence, kv head)); it must lie
 * in [B * H_kv, B * H_kv * cie_paged_decode_max_splits()] and be a multiple
 * of H_kv.  Equal lengths give every (sequence, kv head) n_workgroups /
 * (B * H_kv) splits; unequal ones give longer sequences more.  partials:
 * cie_paged_decode_planned_partials_bytes(n_workgroups, H_q, H_kv, D);
 * counters: 2 * B * H_kv words as for cie_paged_decode.  B <= 1024.
 * Replaces decode_gqa_attention (attn/core.py:13-66) and its grid
 * (P, H_kv, B) (attn/core.py:37) for every layer of a decode step.
 */
int64_t cie_paged_decode_plan_workgroups(int64_t B, int64_t H_kv, int64_t n_splits);
int64_t cie_paged_decode_plan_bytes(int64_t n_workgroups);
int64_t cie_paged_decode_planned_partials_bytes(int64_t n_workgroups, int64_t H_q, int64_t H_kv,
                                                int64_t D);
int cie_paged_decode_plan(void* plan, const int64_t* lens, const int64_t* slot_ids,
                          const int64_t* block_table, int64_t B, int64_t H_kv,
                          int64_t page_size, int64_t n_pages, int64_t bt_stride,
                          int64_t bt_width, int64_t n_slots, int64_t append,
                          int64_t n_workgroups, int32_t* err, void* stream);
int cie_paged_decode_planned(void* o, const void* q, const void* k_pool, const void* v_pool,
                             const int32_t* plan, const int64_t* block_table, void* partials,
                             int32_t* counters, int64_t B, int64_t H_q, int64_t H_kv, int64_t D,
                             int64_t page_size, int64_t n_pages, int64_t pool_page_stride,
                             int64_t pool_head_stride, int64_t bt_stride, int64_t bt_width,
                             int64_t n_workgroups, int32_t* err, void* stream);
int cie_paged_decode_append_planned(void* o, const void* q, void* k_pool, void* v_pool,
                                    const void* k_new, const void* v_new,
                                    int64_t k_tok_stride, int64_t k_head_stride,
                                    int64_t v_tok_stride, int64_t v_head_stride,
                                    const int32_t* plan, const int64_t* block_table,
                                    void* partials, int32_t* counters,
                                    int64_t B, int64_t H_q, int64_t H_kv, int64_t D,
                                    int64_t page_size, int64_t n_pages,
                                    int64_t pool_page_stride, int64_t pool_head_stride,
                                    int64_t bt_stride, int64_t bt_width, int64_t n_workgroups,
                                    int32_t* err, void* stream);
int cie_paged_decode_qkv_rope_planned(void* o, const void* qkv, int64_t qkv_row_stride,
                                      const void* cos, const void* sin, int64_t cs_row_stride,
                                      void* k_pool, void* v_pool, const int32_t* plan,
                                      const int64_t* block_table, void* partials,
                                      int32_t* counters, int64_t B, int64_t H_q, int64_t H_kv,
                                      int64_t D, int64_t page_size, int64_t n_pages,
                                      int64_t pool_page_stride, int64_t pool_head_stride,
                                      int64_t bt_stride, int64_t bt_width, int64_t n_workgroups,
                                      int32_t* err, void* stream);

/*
 * Allocation-free form of cie_paged_decode_append.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * hipGraph stream capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and result as cie_paged_decode_append without
 * `partials` / `counters`: those live in a static device array of this
 * library (4 MiB of split partials plus 16,384 counter words, one copy per
 * GPU, held until the process ends).  The counters are zeroed by a fill
 * kernel on `stream` at the first call on a device and left zero by every
 * completed call.  A call with n_splits > 1 whose partials
 * (cie_paged_decode_partials_bytes) exceed 4 MiB or with 2 * B * H_kv > 16384
 * returns CIE_ESCRATCH and launches nothing (a one-split call uses no
 * scratch).  cie_paged_decode_noalloc_limit(H_q, H_kv, D, n_splits) gives the
 * largest B this entry point accepts (the scratch bounds, and the kernel's
 * B <= 65535), or -1 for arguments no call accepts (n_splits outside
 * [1, cie_paged_decode_max_splits()], H_q not a multiple of H_kv).  Every
 * call on one GPU shares the array: calls that can overlap in time on one
 * GPU (different streams) race and must not be made.
 */
int64_t cie_paged_decode_noalloc_limit(int64_t H_q, int64_t H_kv, int64_t D, int64_t n_splits);
int cie_paged_decode_append_noalloc(void* o, const void* q, void* k_pool, void* v_pool,
                                    const void* k_new, const void* v_new,
                                    int64_t k_tok_stride, int64_t k_head_stride,
                                    int64_t v_tok_stride, int64_t v_head_stride,
                                    const int64_t* lens, const int64_t* slot_ids,
                                    const int64_t* block_table,
                                    int64_t B, int64_t H_q, int64_t H_kv, int64_t D,
                                    int64_t page_size, int64_t n_pages,
                                    int64_t pool_page_stride, int64_t pool_head_stride,
                                    int64_t bt_stride, int64_t bt_width,
                                    int64_t n_slots, int64_t n_splits, int32_t* err,
                                    void* stream);

/*
 * Decode step from the fused QKV projection, RoPE and KV append fused in, one
 * launch.  Row b of qkv (qkv_row_stride elements apart, 16-byte aligned)
 * holds q (H_q heads), then k (H_kv), then v (H_kv), D each; cos / sin rows b
 * (cs_row_stride apart) are the new token's rotary tables.  q and k are
 * rotated in registers as transformers' apply_rotary_pos_emb does
 * (x*cos + rotate_half(x)*sin, computed in fp32, rounded once to fp16), the
 * rotated k and v rows are appended at pos = lens[slot_ids[b]], and o is the
 * decode attention of the rotated q over the pos + 1 tokens.
 * Replaces the decode branch of TritonQwen2Attention.forward
 * (attn/core.py:181-215): the QKV split, apply_rotary_pos_emb,
 * KVStorage.decode_update and gqa_decode_attention.  Other arguments as for
 * cie_paged_decode_append.
 */
int cie_paged_decode_qkv_rope(void* o, const void* qkv, int64_t qkv_row_stride,
                              const void* cos, const void* sin, int64_t cs_row_stride,
                              void* k_pool, void* v_pool,
                              const int64_t* lens, const int64_t* slot_ids,
                              const int64_t* block_table, void* partials,
                              int32_t* counters,
                              int64_t B, int64_t H_q, int64_t H_kv, int64_t D,
                              int64_t page_size, int64_t n_pages,
                              int64_t pool_page_stride, int64_t pool_head_stride,
                              int64_t bt_stride, int64_t bt_width, int64_t n_slots,
                              int64_t n_splits, int32_t* err, void* stream);

/*
 * Token-mode append from the fused QKV projection, with RoPE: for each packed
 * token t < T (row t of qkv, layout as for cie_paged_decode_qkv_rope; cos /
 * sin row t), the rotated q heads go to q_out (T, H_q, D) dense, and the
 * rotated k and the v rows to (pages[t], head, offsets[t]) of the pools.
 * Replaces the mixed branch's QKV split, apply_rotary_pos_emb and
 * KVStorage.mixed_update (attn/core.py:181-198, 226-229;
 * kv_cache/storage.py:62-85).  D must be a multiple of 16; every pointer
 * 16-byte aligned.
 */
int cie_kv_append_tokens_qkv_rope(void* q_out, void* k_pool, void* v_pool,
                                  const void* qkv, int64_t qkv_row_stride,
                                  const void* cos, const void* sin,
                                  int64_t cs_row_stride,
                                  const int64_t* pages, const int64_t* offsets,
                                  int64_t T, int64_t H_q, int64_t H_kv,
                                  int64_t page_size, int64_t D, int64_t n_pages,
                                  int64_t pool_page_stride,
                                  int64_t pool_head_stride, int32_t* err,
                                  void* stream);

/*
 * Varlen causal GQA attention over the paged pool for a packed batch of
 * chunked-prefill and decode sequences.  Sequence b owns query rows
 * [cu_seqlens[b], cu_seqlens[b+1]); its row i sits at absolute position
 * kv_lens[b] + i and attends keys [0, kv_lens[b] + i] of slot slot_ids[b].
 * Rows outside every sequence are not written.
 * Replaces mixed_gqa_attention (attn/core.py:69-111), i.e. the Triton
 * mixed_gqa_attention_kernel (kernels/prefill_attention.py:10-198).
 *   q, o       : (total_T, H_q, D) dense fp16
 *   max_seqlen : upper bound on every sequence's query length (the
 *                reference's metadata token-count bucket); rows past it are
 *                not computed (CIE_ERRBIT_LEN).  B <= 1024 (its plan
 *                tables live in LDS: a batch that would take a workgroup
 *                past the device's LDS limit gets CIE_EUNSUPPORTED).
 *   partials, partials_bytes : a 16-byte aligned buffer of any contents
 *                (per-chunk softmax state of the tiles the call splits over
 *                several workgroups); its size is a budget, not a bound the
 *                call checks against the batch.  Sequences whose split
 *                tiles' rows (rows x H_q x chunks of each split tile) fit
 *                the budget, in sequence order, are split; the rest run
 *                unsplit — same results, longer critical path.  A row takes
 *                4 * (D + 2) bytes; the budget caps at 2,097,088 rows.
 *                cie_mixed_partials_bytes(total_T, H_q, D) is the default:
 *                per q head, the larger of 2 rows per token and 16 rows (a
 *                decode row's most chunks) for each of the first 64 tokens
 *                (about 7.8 MB for 1,052 tokens, 14 heads, D = 64; 3.8 MB
 *                at most below 512 tokens); partials may be NULL with
 *                partials_bytes = 0 (nothing splits).
 *   counters   : cie_mixed_counters(B, H_kv, max_seqlen) int32, 16-byte
 *                aligned, zero before the call and left zero by it (an
 *                arrival word and a stale word per query tile and column
 *                group, with CIE_ERRBIT_SPLIT as for cie_paged_decode; the
 *                same buffer can serve cie_paged_decode, calls being
 *                stream-ordered)
 */
int64_t cie_mixed_partials_bytes(int64_t total_T, int64_t H_q, int64_t D);
int64_t cie_mixed_counters(int64_t B, int64_t H_kv, int64_t max_seqlen);
int cie_mixed_attention(void* o, const void* q,
                        const void* k_pool, const void* v_pool,
                        const int64_t* cu_seqlens, const int64_t* kv_lens,
                        const int64_t* slot_ids, const int64_t* block_table,
                        void* partials, int64_t partials_bytes, int32_t* counters,
                        int64_t B, int64_t total_T, int64_t max_seqlen,
                        int64_t H_q, int64_t H_kv, int64_t D,
                        int64_t page_size, int64_t n_pages,
                        int64_t pool_page_stride, int64_t pool_head_stride,
                        int64_t bt_stride, int64_t bt_width, int64_t n_slots,
                        int32_t* err, void* stream);

/*
 * Planned mixed attention: one plan per mixed step.  The batch's sequences
 * (cu_seqlens, kv_lens, slot_ids) are the same for every layer of a step, as
 * the reference's AttentionMetadata is built once per step
 * (attn/metadata.py:3-55) and every layer's mixed_gqa_attention reads it
 * (attn/core.py:69-111).  cie_mixed_plan runs the plan each launch of
 * cie_mixed_attention makes for itself — the work items, their order and
 * the sequences' partial bases — once, into `plan`; each layer's
 * cie_mixed_attention_planned then reads its items' descriptors in one
 * memory round trip instead of loading the sequence tables and planning.
 * The results equal cie_mixed_attention's bit for bit.
 *   plan          : cie_mixed_plan_bytes(B, total_T) bytes, 16-byte aligned;
 *                   valid for the batch (cu_seqlens, kv_lens, slot_ids),
 *                   shape and partials_bytes it was made with.  A planned
 *                   call whose B, max_seqlen's query tiles, H_q, H_kv or
 *                   partials budget differ from the plan's writes nothing
 *                   and raises CIE_ERRBIT_PLAN.  A batch with more items than
 *                   the plan holds (only sequences that overlap in
 *                   cu_seqlens can have them) gets an empty plan and
 *                   CIE_ERRBIT_PLAN.  Rows past max_seqlen are reported
 *                   (CIE_ERRBIT_LEN) by cie_mixed_plan.
 *   other arguments as for cie_mixed_attention.
 */
int64_t cie_mixed_plan_bytes(int64_t B, int64_t total_T);
int cie_mixed_plan(int32_t* plan, int64_t plan_bytes,
                   const int64_t* cu_seqlens, const int64_t* kv_lens, const int64_t* slot_ids,
                   int64_t B, int64_t total_T, int64_t max_seqlen,
                   int64_t H_q, int64_t H_kv, int64_t D, int64_t page_size,
                   int64_t bt_width, int64_t n_slots, int64_t partials_bytes,
                   int32_t* err, void* stream);
int cie_mixed_attention_planned(void* o, const void* q,
                                const void* k_pool, const void* v_pool,
                                const int32_t* plan, int64_t plan_bytes,
                                const int64_t* block_table,
                                void* partials, int64_t partials_bytes, int32_t* counters,
                                int64_t B, int64_t total_T, int64_t max_seqlen,
                                int64_t H_q, int64_t H_kv, int64_t D,
                                int64_t page_size, int64_t n_pages,
                                int64_t pool_page_stride, int64_t pool_head_stride,
                                int64_t bt_stride, int64_t bt_width, int64_t n_slots,
                                int32_t* err, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CIE_PAGED_ATTENTION_H */
