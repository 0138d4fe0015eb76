/*
 * crane_kv.h -- C ABI of the host-side KV-cache manager above crane_hip.h.
 *
 * One crane_kv object is one attention layer's K/V cache pair in Crane's
 * layout, [B, Hkv, cap, D] with rows of D contiguous, plus the number of valid
 * rows of every sequence (kept on the host and on the device).  It replaces:
 *
 *   crane_kv_update / crane_kv_append_qkv   Attention::update_kv_cache
 *       (qwen3/modeling.rs:313-370, hunyuan_dense/modeling.rs:433-489): rows are
 *       written in place while they fit; on the first use the buffer is
 *       allocated with S + 256 rows, and when it is full it is reallocated
 *       with (rows needed) + 256 rows and the valid rows copied over
 *       (crane_kv_grown_capacity states the policy).
 *   crane_kv_stack     Qwen3Model::setup_batch_decode + pad_and_stack_kv_caches
 *       (qwen3/modeling.rs:973-1030, 1141-1200): N single-sequence caches are
 *       copied into one batch cache.  Sequence i's rows start at row 0 and
 *       its length is kept, instead of right-aligned padding and a -1e9 mask;
 *       the decode kernel reads exactly len[i] rows, which gives the same
 *       softmax (exp(-1e9 - m) == 0 in f32).
 *   crane_kv_extract   Qwen3Model::extract_batch_kv (:1066-1102): sequence i's
 *       valid rows copied out into a single-sequence cache.
 *   crane_kv_bytes     Qwen3Model::active_kv_cache_bytes (:912-929): bytes of
 *       the allocated K and V buffers.
 *   crane_kv_views     get_kv_caches (:937-952): device pointers of the buffers
 *       and the valid lengths (the views a caller narrows to len rows).
 *   crane_kv_set_lengths  set_kv_caches (:954-966) for an existing buffer.
 *
 * Conventions are those of crane_hip.h: 0 or a CRANE_HIP_E_* status, checked
 * on the host before anything is enqueued; everything is ordered on `stream`.
 * Unlike the kernel launchers, these functions allocate and free device memory
 * (hipMalloc / hipFree), as candle's tensor ops do; a reallocation synchronises
 * the stream before freeing the old buffer.  Rows at or past a sequence's
 * length are never read and their contents are unspecified (candle's buffers
 * hold zeros there).  One object must not be used from two threads at once.
 */
#ifndef CRANE_KV_H
#define CRANE_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct crane_kv crane_kv;

/* Crane's growth room: rows added beyond what is needed on (re)allocation. */
#define CRANE_KV_ROOM 256

/* The capacity a cache of `cap` rows has after making room for `needed` rows:
 * `cap` when needed <= cap, else needed + CRANE_KV_ROOM (first use included).
 * Host-only, no side effects; -1 for negative arguments. */
int64_t crane_kv_grown_capacity(int64_t cap, int64_t needed);

/* A cache for B sequences of Hkv heads of D (= 128) in `dtype`, with no buffer
 * yet (capacity 0, every length 0). */
int crane_kv_create(int B, int Hkv, int D, int dtype, crane_kv** out);
void crane_kv_destroy(crane_kv* kv);

/* Ensure every sequence has room for `add_rows` more rows (the policy above,
 * applied to the longest sequence). */
int crane_kv_reserve(crane_kv* kv, int64_t add_rows, void* stream);

/* Attention::update_kv_cache: append k, v [B, Hkv, S, D] (contiguous, in the
 * cache dtype) at every sequence's length; lengths grow by S. */
int crane_kv_update(crane_kv* kv, const void* k, const void* v, int S, void* stream);

/* The fused path: reserve S rows, run crane_hip_qknorm_rope_append into this
 * cache at the current lengths (token s of sequence b at table row
 * positions[b] + s), then lengths grow by S.  Arguments as in crane_hip.h. */
int crane_kv_append_qkv(crane_kv* kv, const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                        const void* k_norm_w, float eps, int order, const void* cos, const void* sin,
                        int64_t cs_stride, int64_t table_rows, const int32_t* positions, void* q_out, int S,
                        int Hq, void* stream);

/* Decode over the cache (crane_hip_attn_decode with kv_len = the lengths;
 * score_mode as there). */
int crane_kv_decode(const crane_kv* kv, const void* q, int Hq, float scale, int score_mode, void* workspace,
                    size_t ws_bytes, void* out, void* stream);

/* Causal or full prefill of the last S rows of every sequence (queries q
 * [B, Hq, S, D]; sequence b's chunk starts at row len[b] - S).  flags: the
 * CRANE_HIP_PREFILL_* bits of crane_hip_attn_prefill (1 = causal). */
int crane_kv_prefill(const crane_kv* kv, const void* q, int Hq, int S, float scale, int flags, void* out,
                     void* stream);

/* Device pointers of the K and V buffers (NULL before the first use), the
 * capacity in rows, the device array of lengths (int32 [B]) and a host copy
 * of the lengths (int64, B entries written to host_len when non-NULL). */
int crane_kv_views(const crane_kv* kv, void** k, void** v, int64_t* cap, const int32_t** dev_len,
                   int64_t* host_len);

/* Set the lengths of an existing buffer (set_kv_caches); each <= capacity. */
int crane_kv_set_lengths(crane_kv* kv, const int64_t* host_len, void* stream);

/* Bytes of the allocated K and V buffers (0 before the first use). */
uint64_t crane_kv_bytes(const crane_kv* kv);

/* Batched decode set-up: `dst` (B = n, same Hkv, D, dtype; any prior buffer is
 * released) receives a buffer of max_i(len_i) + extra_room rows and the rows
 * of srcs[i] (each B = 1) at rows [0, len_i) of sequence i.  No srcs[i] may be
 * dst itself (CRANE_HIP_E_INVALID: its rows would be released first). */
int crane_kv_stack(crane_kv* dst, const crane_kv* const* srcs, int n, int64_t extra_room, void* stream);

/* Batched decode tear-down: copy sequence i of `batch` (its len_i rows) into
 * `dst` (B = 1, same Hkv, D, dtype).  A dst buffer smaller than len_i rows is
 * replaced by one of exactly len_i rows, as extract_batch_kv's contiguous
 * copies are; the next append then grows it by the policy above. */
int crane_kv_extract(const crane_kv* batch, int i, crane_kv* dst, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CRANE_KV_H */
