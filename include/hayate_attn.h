/*
 * hayate_attn.h — C ABI of the MI355X (gfx950) paged-attention library
 * libhayate_attn.so.
 *
 * Every entry point takes raw device pointers, element strides (int64, in
 * elements, not bytes), int32 metadata and a hipStream_t (passed as void* so
 * this header needs no HIP include). Nothing here allocates device memory:
 * all buffers, including the split-K workspace, belong to the caller.
 * Functions enqueue asynchronously on the given stream, never synchronise,
 * and return 0 on success or a negative HY_E* code; hy_last_error() then
 * returns a message for the calling thread.
 *
 * KV pool layout (one transformer layer, as in the reference's pool tensors
 * of shape (layers, 1, kv_heads, capacity, head_dim), hayate/engine/
 * paged_cache.py:104-109): element (h, p, d) of a layer lives at
 *   base + h * pool_head_stride + p * head_dim + d
 * with physical token p = page_id * page_size + offset.
 *
 * Query/key/value/output rows are addressed per sequence b, token i within
 * that sequence and head h as
 *   base + b * stride_seq + (q_start[b] + i) * stride_tok + h * stride_head
 * so both a padded (B, H, T, D) view and a packed varlen (N, H, D) tensor
 * can be passed without a copy. q_start has num_seqs + 1 entries
 * (cumulative query lengths, q_start[0] == 0).
 *
 * Supported geometry: head_dim == 128, page_size a power of two >= 32,
 * num_q_heads / num_kv_heads in {1, 2, 4, 8, 16}; bf16 storage.
 */
#ifndef HAYATE_ATTN_H
#define HAYATE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HY_OK 0
#define HY_EINVAL (-1)       /* invalid argument (shape, null pointer, range) */
#define HY_ELAUNCH (-2)      /* HIP launch or runtime error */
#define HY_EUNSUPPORTED (-3) /* geometry the kernels are not built for */
#define HY_ENOSPACE (-4)     /* caller buffer too small */

/* Library version, (major << 16) | minor. No reference counterpart. */
int hy_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char *hy_last_error(void);

/*
 * Paged KV append: pool[h, phys(b, c_b + i)] = k[b, i, h] (and v), a pure
 * bit copy, for every sequence b < num_seqs, token i < q_len_b and kv head h.
 * phys(b, t) = page_table[b * page_table_stride + t / page_size] * page_size
 *              + t % page_size, c_b = cache_lens[b].
 * Replaces PagedKVBatch.write_layer (hayate/engine/paged_cache.py:44-60).
 */
int hy_kv_append(void *k_pool, void *v_pool, int64_t pool_head_stride,
                 const void *k, int64_t k_stride_seq, int64_t k_stride_tok,
                 int64_t k_stride_head, const void *v, int64_t v_stride_seq,
                 int64_t v_stride_tok, int64_t v_stride_head,
                 const int32_t *q_start, const int32_t *cache_lens,
                 const int32_t *page_table, int64_t page_table_stride,
                 int32_t num_seqs, int32_t total_tokens, int32_t num_kv_heads,
                 int32_t head_dim, int32_t page_size, void *stream);

/*
 * Fused per-head RMSNorm + rotary embedding of q and k, then paged append of
 * k and v. For token i of sequence b at position pos = cache_lens[b] + i:
 *   x' = bf16((x * (1 / sqrt(mean(x^2) + eps))) * w)          (fp32 math)
 * with eps = q_eps for q rows and k_eps for k rows (the two RMSNorm modules
 * of attention.py:34-35 each carry their own eps).
 *   y  = bf16(x' * cos[pos] + rotate_half(x') * sin[pos])       (fp32 math)
 * q' goes to q_out; k' and v (unchanged) are appended as hy_kv_append does.
 * q_norm_weight / k_norm_weight may be NULL (no norm); cos_table/sin_table
 * may be NULL (no rotation); tables are fp32 (max_positions, head_dim).
 * Every position cache_lens[b] + i must be below max_positions: this is the
 * caller's guarantee (the kernels clamp the table row so that a call which
 * breaks it cannot read past the tables, but its rotation is then wrong).
 * Replaces GroupedQueryAttention.forward lines 62-75 (hayate/model/
 * attention.py:62-75: q_norm, k_norm, apply_rope_vectorized, write_layer),
 * with hayate/model/rope.py:31-47 for the rotation.
 */
int hy_qknorm_rope_append(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
    int64_t q_stride_head, void *q_out, int64_t qo_stride_seq,
    int64_t qo_stride_tok, int64_t qo_stride_head, const void *k,
    int64_t k_stride_seq, int64_t k_stride_tok, int64_t k_stride_head,
    const void *v, int64_t v_stride_seq, int64_t v_stride_tok,
    int64_t v_stride_head, const void *q_norm_weight,
    const void *k_norm_weight, float q_eps, float k_eps,
    const float *cos_table,
    const float *sin_table, int32_t max_positions, void *k_pool, void *v_pool,
    int64_t pool_head_stride, const int32_t *q_start,
    const int32_t *cache_lens, const int32_t *page_table,
    int64_t page_table_stride, int32_t num_seqs, int32_t total_tokens,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, void *stream);

/*
 * Page gather: out[l, h, t, :] = pool[l, h, phys(t), :] for t < length over
 * the given page list, out contiguous (num_layers, num_kv_heads, length,
 * head_dim). A bit copy. Replaces PagedKVCacheManager.snapshot's
 * index_select (hayate/engine/paged_cache.py:180-190, 306-315).
 */
int hy_page_gather(const void *pool, int64_t pool_layer_stride,
                   int64_t pool_head_stride, const int32_t *pages,
                   int32_t length, void *out, int32_t num_layers,
                   int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                   void *stream);

/*
 * Page scatter, the inverse of hy_page_gather: pool[l, h, phys(t), :] =
 * src[l, h, t, :] with src strided (layer, head, token). Replaces
 * PagedKVCacheManager.import_cache's index_copy_ (paged_cache.py:153-166).
 */
int hy_page_scatter(void *pool, int64_t pool_layer_stride,
                    int64_t pool_head_stride, const int32_t *pages,
                    int32_t length, const void *src, int64_t src_stride_layer,
                    int64_t src_stride_head, int64_t src_stride_tok,
                    int32_t num_layers, int32_t num_kv_heads,
                    int32_t head_dim, int32_t page_size, void *stream);

/*
 * Tick planner (host only, no device access). Given per-sequence query
 * lengths and KV lengths (kv_len = cache_len + q_len), split the work of
 * one attention call into:
 *   decode items  (q_len == 1): int32[n_chunks + n_pieces][8]. The K/V
 *                 rows of all decode sequences, in sequence order, form one
 *                 token stream per kv head, cut into n_chunks chunks of
 *                 equal length (one workgroup each; a cut inside a sequence
 *                 falls on a multiple of 32 of its tokens). A piece is the
 *                 part of one sequence inside one chunk. The first n_chunks
 *                 records are chunks {piece_begin, piece_end, n_slices, and
 *                 the first piece's seq, tok_begin, tok_end, slot_base,
 *                 q_row}; the piece records follow: {seq, tok_begin,
 *                 tok_end, slot_base, slice_begin, q_row, q_pos, ends}, where
 *                 slot_base = W * piece index (W partials per piece, one per
 *                 wave), slice_begin counts 32-token slices from the start
 *                 of the chunk, q_row is the sequence's packed query row
 *                 (the prefix sum of q_lens), q_pos = kv_len - 1 the
 *                 position of its query token and ends = 1 for the piece
 *                 that holds that position;
 *   merge items   int32[n][4] = {seq, first_slot, num_partials, q_row}, one
 *                 per decode sequence (all of its pieces' partials);
 *   prefill items (q_len > 1): int32[n][8] =
 *                 {seq, q_begin, q_end, kv_begin, kv_end, slot, q_row,
 *                 cache_len}: query tiles of 256 / G tokens, each over one
 *                 range of keys (kv_begin a multiple of 64), most keys
 *                 first; slot as for decode items, q_row as for decode
 *                 pieces, cache_len = kv_len - q_len of the sequence;
 *   prefill merge items int32[n][8] =
 *                 {seq, q_begin, q_end, first_slot, num_splits, q_row, 0, 0}.
 * Decode uses one chunk per CU and kv head (num_cus / num_kv_heads chunks,
 * at least 64 tokens each); a chunk also ends after as many pieces as the
 * kernel's query table holds. Prefill split lengths are chosen by
 * simulating the longest-first dispatch of the work onto num_cus CUs.
 * counts_out (int32[7]) receives {n_chunks, n_merge, n_decode_slots,
 * n_prefill, n_prefill_merge, n_prefill_slots, n_pieces}. Capacities are in
 * items (decode: chunk + piece records); returns HY_ENOSPACE if one is too
 * small. target_tokens_per_split > 0 sets the decode chunk length instead.
 * Replaces the per-forward metadata of PagedKVCacheManager.begin_batch
 * (paged_cache.py:202-293: page table, cache_lens, kv_lens, block mask).
 */
int hy_plan_tick(const int32_t *q_lens, const int32_t *kv_lens,
                 int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                 int32_t page_size, int32_t num_cus,
                 int32_t target_tokens_per_split, int32_t *decode_items,
                 int32_t decode_capacity, int32_t *merge_items,
                 int32_t merge_capacity, int32_t *prefill_items,
                 int32_t prefill_capacity, int32_t *prefill_merge_items,
                 int32_t prefill_merge_capacity, int32_t *counts_out);

/* Split-K workspace bytes for n_slots fp32 partials (acc[head_dim], max,
 * sum per query head). */
int64_t hy_decode_workspace_bytes(int32_t n_slots, int32_t num_q_heads,
                                  int32_t head_dim);

/*
 * Paged GQA decode attention for sequences with one query token each
 * (decode items from hy_plan_tick; n_decode = n_chunks). Each workgroup
 * covers one chunk and one kv head, loads every K/V row of its pieces once
 * and applies it to all num_q_heads / num_kv_heads query heads (QK^T and
 * PV on MFMA). Every piece leaves fp32 partials in the workspace;
 * hy_paged_decode_merge, enqueued after this call on the same stream,
 * writes the output rows (out and q_start are validated here but written
 * and read by the merge).
 * Causal semantics: the query of sequence b at position kv_len - 1 sees
 * every key k < kv_len (paged_cache.py:266-271). n_decode is at most 65535
 * (the grid's y limit); more returns HY_EINVAL. The chunk records may be
 * followed by empty ones (piece_begin == piece_end) up to n_decode, which
 * do nothing: a caller that captures the launch in a graph can pass a fixed
 * n_decode and pad the plan's records (the piece records then start after
 * all n_decode chunk records).
 * Replaces PagedKVBatch.attend_layer (paged_cache.py:62-71) for T == 1.
 */
int hy_paged_decode(const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
                    int64_t q_stride_head, void *out, int64_t o_stride_seq,
                    int64_t o_stride_tok, int64_t o_stride_head,
                    const void *k_pool, const void *v_pool,
                    int64_t pool_head_stride, const int32_t *page_table,
                    int64_t page_table_stride, const int32_t *q_start,
                    const int32_t *decode_items, int32_t n_decode,
                    int32_t n_slots, void *workspace, int64_t workspace_bytes,
                    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                    int32_t head_dim, int32_t page_size, float scale,
                    void *stream);

/*
 * hy_qknorm_rope_append fused into hy_paged_decode for a batch whose
 * sequences all have q_len == 1 (every sequence's token is appended at
 * position cache_lens[b] and attends to keys 0 .. cache_lens[b]). q, k, v
 * are the raw projections with the strides of hy_qknorm_rope_append; the
 * rotated q rows are written to q_out, the new K and V rows to their pages,
 * bit-identical to hy_qknorm_rope_append, and the attention partials to the
 * workspace as hy_paged_decode does (hy_paged_decode_merge then writes out).
 * As for hy_qknorm_rope_append, cache_lens[b] < max_positions is the
 * caller's guarantee.
 * One launch instead of two per decode layer: the workgroups rotate the
 * query rows of their pieces themselves and take the new token's K/V row
 * from LDS, so no workgroup waits for another's write.
 * Replaces the decode case of attention.py:62-75 (norm, rope, write_layer)
 * followed by paged_cache.py:62-71 (attend_layer).
 */
int hy_paged_decode_append(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
    int64_t q_stride_head, void *q_out, int64_t qo_stride_seq,
    int64_t qo_stride_tok, int64_t qo_stride_head, const void *k,
    int64_t k_stride_seq, int64_t k_stride_tok, int64_t k_stride_head,
    const void *v, int64_t v_stride_seq, int64_t v_stride_tok,
    int64_t v_stride_head, const void *q_norm_weight,
    const void *k_norm_weight, float q_eps, float k_eps,
    const float *cos_table,
    const float *sin_table, int32_t max_positions, void *out, void *k_pool,
    void *v_pool, int64_t pool_head_stride, const int32_t *page_table,
    int64_t page_table_stride, const int32_t *q_start,
    const int32_t *cache_lens, const int32_t *decode_items, int32_t n_decode,
    int32_t n_slots, void *workspace, int64_t workspace_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t page_size, float scale, void *stream);

/*
 * Merge of split decode partials (log-sum-exp over the splits of each
 * merge item) into the bf16 output rows of hy_paged_decode. Second half of
 * PagedKVBatch.attend_layer (paged_cache.py:62-71) for split sequences.
 */
int hy_paged_decode_merge(void *out, int64_t o_stride_seq, int64_t o_stride_tok,
                          int64_t o_stride_head, const int32_t *q_start,
                          const int32_t *merge_items, int32_t n_merge,
                          int32_t n_slots, const void *workspace,
                          int64_t workspace_bytes, int32_t num_q_heads,
                          int32_t head_dim, void *stream);

/* Size of the static device scratch of hy_paged_decode_append_noalloc, per
 * GPU (8 MiB: the partials of 252 pieces at 32 query heads; the batch-32
 * decode step needs about 2 MB). */
#define HY_NOALLOC_SCRATCH_BYTES (8 * 1024 * 1024)

/*
 * hy_paged_decode_append followed by hy_paged_decode_merge, with the split
 * partials in a static device array of HY_NOALLOC_SCRATCH_BYTES owned by the
 * library instead of a caller workspace: a call allocates nothing (no
 * hipMalloc, no allocating library routine). No counterpart in the
 * reference: it is for callers that cannot allocate device memory — code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation. Arguments are those of the two calls it combines (out strides
 * and merge items of hy_paged_decode_merge; no workspace). Returns
 * HY_ENOSPACE when hy_decode_workspace_bytes(n_slots, num_q_heads, head_dim)
 * exceeds HY_NOALLOC_SCRATCH_BYTES. Each GPU holds one array for the life of
 * the process, shared by every call on that GPU and keeping the last call's
 * contents: calls that overlap on one GPU (several streams or threads) race.
 */
int hy_paged_decode_append_noalloc(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
    int64_t q_stride_head, void *q_out, int64_t qo_stride_seq,
    int64_t qo_stride_tok, int64_t qo_stride_head, const void *k,
    int64_t k_stride_seq, int64_t k_stride_tok, int64_t k_stride_head,
    const void *v, int64_t v_stride_seq, int64_t v_stride_tok,
    int64_t v_stride_head, const void *q_norm_weight,
    const void *k_norm_weight, float q_eps, float k_eps,
    const float *cos_table,
    const float *sin_table, int32_t max_positions, void *out,
    int64_t o_stride_seq, int64_t o_stride_tok, int64_t o_stride_head,
    void *k_pool, void *v_pool, int64_t pool_head_stride,
    const int32_t *page_table, int64_t page_table_stride,
    const int32_t *q_start, const int32_t *cache_lens,
    const int32_t *decode_items, int32_t n_decode, const int32_t *merge_items,
    int32_t n_merge, int32_t n_slots, int32_t num_seqs, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, float scale,
    void *stream);

/* (token, head) rows of one prefill query tile: hy_plan_tick cuts prefill
 * sequences into tiles of hy_prefill_tile_rows() / G tokens (G = query heads
 * per kv head), so callers size the prefill item list from it. Part of the
 * work-list format that replaces the reference's BlockMask blocks
 * (hayate/engine/paged_cache.py:273-284); no reference counterpart. */
int32_t hy_prefill_tile_rows(void);

/* Prefill split workspace bytes for n_slots partials (fp32 acc[head_dim],
 * max, sum for each of the hy_prefill_tile_rows() rows of a query tile, per
 * kv head). */
int64_t hy_prefill_workspace_bytes(int32_t n_slots, int32_t num_kv_heads,
                                   int32_t head_dim);

/*
 * Paged chunked-prefill causal attention (bf16 MFMA) for sequences with
 * q_len > 1 (prefill items from hy_plan_tick): query i of sequence b at
 * logical position cache_len_b + i sees every cached prefix key and the
 * chunk's keys up to itself. K/V are read through the page table. Split
 * query tiles leave fp32 partials in the workspace; hy_paged_prefill_merge,
 * enqueued after this call on the same stream, completes them. A record
 * with q_end <= q_begin (prefill) or num_splits == 0 (merge) is empty and
 * skipped, so a caller can pad both lists to a fixed launch size (a
 * captured graph's). n_prefill (and n_merge of the merge) is at most 65535
 * (the grid's y limit); more returns HY_EINVAL.
 * Replaces PagedKVBatch.attend_layer (paged_cache.py:62-71) for T > 1.
 */
int hy_paged_prefill(const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
                     int64_t q_stride_head, void *out, int64_t o_stride_seq,
                     int64_t o_stride_tok, int64_t o_stride_head,
                     const void *k_pool, const void *v_pool,
                     int64_t pool_head_stride, const int32_t *page_table,
                     int64_t page_table_stride, const int32_t *q_start,
                     const int32_t *kv_lens, const int32_t *prefill_items,
                     int32_t n_prefill, int32_t n_slots, void *workspace,
                     int64_t workspace_bytes, int32_t num_seqs,
                     int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t page_size, float scale,
                     void *stream);

/*
 * Merge of split prefill partials into the bf16 output rows of
 * hy_paged_prefill (one merge item per split query tile).
 */
int hy_paged_prefill_merge(void *out, int64_t o_stride_seq, int64_t o_stride_tok,
                           int64_t o_stride_head, const int32_t *q_start,
                           const int32_t *merge_items, int32_t n_merge,
                           int32_t n_slots, const void *workspace,
                           int64_t workspace_bytes, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim,
                           void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HAYATE_ATTN_H */
