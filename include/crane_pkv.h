/*
 * crane_pkv.h -- C ABI of the paged KV-cache manager above crane_hip.h.
 *
 * One crane_pkv object is one attention layer's paged K/V cache: two pools of
 * n_pages pages ([n_pages, Hkv, page_rows, D], see the paged launchers in
 * crane_hip.h), a free list, and up to max_seqs sequences, each a list of at
 * most max_pages_per_seq pages and a length.  A sequence's rows never move:
 * appends fill its last page and then take a page from the free list, and
 * batched decode reads every sequence where it is.  It replaces:
 *
 *   Attention::update_kv_cache (qwen3/modeling.rs:313-370): rows are appended
 *       in place; growth takes pages instead of reallocating the whole buffer
 *       with 256 rows of room and copying it (:333-355).
 *   setup_batch_decode + pad_and_stack_kv_caches (:973-1030, 1141-1200) and
 *       extract_batch_kv (:1066-1102): a batch is a list of sequence ids
 *       (crane_pkv_set_batch uploads B rows of page ids and B lengths); no KV
 *       row is copied to set a batch up or to tear it down.
 *   get_kv_caches / set_kv_caches (:937-966): crane_pkv_read_seq and
 *       crane_pkv_write_seq copy one sequence's rows to / from a contiguous
 *       [Hkv, len, D] buffer.
 *   active_kv_cache_bytes (:912-929): crane_pkv_bytes.
 *
 * Conventions are those of crane_hip.h: 0 or a CRANE_HIP_E_* status, checked
 * on the host before anything is enqueued (a call that fails changes nothing);
 * everything is ordered on `stream`.  crane_pkv_create allocates the pools and
 * tables (hipMalloc) and crane_pkv_destroy frees them; set_batch,
 * read_seq and write_seq synchronise the stream after their small uploads; the
 * other calls neither allocate nor synchronise.  Pool rows outside a
 * sequence's length are unspecified.  One object must not be used from two
 * threads at once.
 */
#ifndef CRANE_PKV_H
#define CRANE_PKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct crane_pkv crane_pkv;

/* Pools of n_pages pages of page_rows rows (a positive multiple of
 * CRANE_HIP_PAGE_ALIGN) for Hkv heads of D (= 128) in `dtype`; room for
 * max_seqs live sequences of up to max_pages_per_seq pages each. */
int crane_pkv_create(int Hkv, int D, int dtype, int page_rows, int64_t n_pages, int max_seqs,
                     int max_pages_per_seq, crane_pkv** out);
void crane_pkv_destroy(crane_pkv* pkv);

/* A new, empty sequence; its id is in [0, max_seqs). */
int crane_pkv_seq_add(crane_pkv* pkv, int* seq_id);
/* Release a sequence: its pages return to the free list.  It must not be in
 * the current batch. */
int crane_pkv_seq_free(crane_pkv* pkv, int seq_id);
/* Valid rows of a live sequence, or -1. */
int64_t crane_pkv_seq_len(const crane_pkv* pkv, int seq_id);
/* Pages on the free list. */
int64_t crane_pkv_free_pages(const crane_pkv* pkv);
/* Bytes of the K and V pools. */
uint64_t crane_pkv_bytes(const crane_pkv* pkv);

/* Make seq_ids[0..B) (distinct live sequences, B <= max_seqs) the batch that
 * the calls below operate on; batch row b is sequence seq_ids[b]. */
int crane_pkv_set_batch(crane_pkv* pkv, const int* seq_ids, int B, void* stream);

/* Attention::update_kv_cache on the batch: append k, v [B, Hkv, S, D]
 * (contiguous, cache dtype) at every sequence's length; lengths grow by S. */
int crane_pkv_update(crane_pkv* pkv, const void* k, const void* v, int S, void* stream);

/* The fused QK-norm + RoPE append on the batch (crane_hip_qknorm_rope_append_paged
 * at the current lengths, then lengths grow by S).  Arguments as in crane_hip.h. */
int crane_pkv_append_qkv(crane_pkv* pkv, const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                         const void* k_norm_w, float eps, int order, const void* cos, const void* sin,
                         int64_t cs_stride, int64_t table_rows, const int32_t* positions, void* q_out, int S,
                         int Hq, void* stream);

/* Decode over the batch's rows (crane_hip_attn_decode_paged, kv_len = the
 * lengths; score_mode as there). */
int crane_pkv_decode(const crane_pkv* pkv, const void* q, int Hq, float scale, int score_mode, void* workspace,
                     size_t ws_bytes, void* out, void* stream);

/* Causal or full prefill of the last S rows of every batch sequence (queries
 * q [B, Hq, S, D]; sequence b's chunk starts at row len[b] - S).  flags: the
 * CRANE_HIP_PREFILL_* bits of crane_hip_attn_prefill (1 = causal). */
int crane_pkv_prefill(crane_pkv* pkv, const void* q, int Hq, int S, float scale, int flags, void* out,
                      void* stream);

/* Copy a live sequence's len rows into k, v [Hkv, len, D] (contiguous). */
int crane_pkv_read_seq(crane_pkv* pkv, int seq_id, void* k, void* v, void* stream);
/* Replace a live sequence's rows by k, v [Hkv, len, D] (contiguous); it must
 * not be in the current batch. */
int crane_pkv_write_seq(crane_pkv* pkv, int seq_id, const void* k, const void* v, int64_t len, void* stream);

/* Device pointers for custom kernels: the pools, the current batch's block
 * table (B rows of table_stride = max_pages_per_seq int32 page ids) and its
 * lengths (int32 [B]). */
int crane_pkv_views(const crane_pkv* pkv, void** k_pool, void** v_pool, const int32_t** block_table,
                    int64_t* table_stride, const int32_t** dev_len);

#ifdef __cplusplus
}
#endif
#endif /* CRANE_PKV_H */
