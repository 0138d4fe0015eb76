/*
 * crane_hip.h -- C ABI of the MI355X (gfx950) attention path for Crane.
 *
 * These launchers replace the candle op chain inside Crane's
 * Attention::forward for Qwen3 / Hunyuan-dense / Qwen2.5-style models:
 *
 *   crane_hip_qknorm_rope_append  replaces  qwen3/modeling.rs:382-423 (qkv narrow,
 *       head reshape/transpose, q_norm/k_norm RmsNorm, candle_nn::rotary_emb::rope)
 *       and :313-370 (update_kv_cache slice_set), hunyuan_dense/modeling.rs:517-557
 *       (rope then norm) and qwen25/qwen2.rs:166-183 (rope only, cache append)
 *   crane_hip_attn_decode         replaces  qwen3/modeling.rs:432-467 (GQA-grouped
 *       decode SDPA: q*scale, q@K^T, +mask, softmax_last_dim, @V) and the
 *       batched-decode pad/mask of :1118-1200 (each sequence reads its own
 *       kv_len rows, which equals right-aligned padding with -1e9 on the pad);
 *       hunyuan_dense/modeling.rs:575-608; qwen2.rs:185-206 (repeat_kv + SDPA)
 *   crane_hip_attn_prefill        replaces  qwen3/modeling.rs:469-502 (expand K/V,
 *       q@K^T*scale, +causal mask of :866-884, softmax, @V, transpose to
 *       [B,S,Hq*D]); hunyuan_dense/modeling.rs:610-645; qwen2.rs:191-211
 *
 * Conventions (mirroring Crane's fused_ops CustomOp1 surface,
 * crane-core/src/fused_ops/cuda_impl.rs:43-195, where a bad shape or dtype is
 * a `bail!` and never a crash):
 *   - every launcher returns 0 on success or a CRANE_HIP_E_* code; argument
 *     checks happen on the host before anything is enqueued;
 *   - all pointers are caller-owned device memory (except where noted);
 *     launchers never allocate and are ordered on `stream` (a hipStream_t,
 *     NULL = the default stream); they keep no state between calls and are
 *     re-entrant;
 *   - dtype: CRANE_HIP_F32 or CRANE_HIP_BF16; the cos/sin tables, q, k, v, the
 *     caches and the outputs all share it (Crane casts its tables to the model
 *     dtype, qwen3/modeling.rs:857-864); arithmetic is f32 throughout;
 *   - head_dim D must be 128 (every supported model family uses 128);
 *   - KV cache layout is Crane's: [B, Hkv, cap, D], rows of D contiguous;
 *   - q head h reads kv head h / (Hq / Hkv) (qwen3/modeling.rs:440, utils.rs:48-58).
 */
#ifndef CRANE_HIP_H
#define CRANE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CRANE_HIP_ABI_VERSION 2

enum crane_hip_dtype { CRANE_HIP_F32 = 0, CRANE_HIP_BF16 = 1 };

/* Order of the per-head ops in the fused append.  Qwen3: RmsNorm then RoPE
 * (qwen3/modeling.rs:410-423); Hunyuan: RoPE then RmsNorm
 * (hunyuan_dense/modeling.rs:541-555); Qwen2.5: RoPE only (qwen2.rs:75-76). */
enum crane_hip_order {
    CRANE_HIP_NORM_THEN_ROPE = 0,
    CRANE_HIP_ROPE_THEN_NORM = 1,
    CRANE_HIP_ROPE_ONLY = 2
};

/* Which of candle's two SDPA forms the decode scores follow (the scores'
 * rounding points differ in the model dtype).  Crane picks the form per call:
 *   GROUPED  -- the GQA-grouped decode of qwen3/modeling.rs:432-467 and
 *               hunyuan_dense/modeling.rs:575-608, taken when n_rep > 1 and
 *               seq_len == 1: q * scale rounded to T (:440-441), then q@K^T
 *               rounded to T;
 *   STANDARD -- the standard SDPA of qwen3/modeling.rs:485-488 (taken for
 *               n_rep == 1), hunyuan_dense/modeling.rs:628-631, and every decode
 *               of candle-transformers qwen2 (qwen25/qwen2.rs:196-197): q@K^T
 *               rounded to T, then * scale rounded to T.
 * In f32 both forms differ only in the last bits of the scores. */
enum crane_hip_score { CRANE_HIP_SCORE_GROUPED = 0, CRANE_HIP_SCORE_STANDARD = 1 };

enum crane_hip_status {
    CRANE_HIP_OK = 0,
    CRANE_HIP_E_INVALID = 1,     /* a size, stride or pointer argument is invalid          */
    CRANE_HIP_E_DTYPE = 2,       /* dtype not f32/bf16                                       */
    CRANE_HIP_E_HEAD_DIM = 3,    /* head_dim other than 128                                  */
    CRANE_HIP_E_GQA = 4,         /* Hq not a multiple of Hkv, or group too large             */
    CRANE_HIP_E_CAPACITY = 5,    /* rows would land past the cache capacity                  */
    CRANE_HIP_E_WORKSPACE = 6,   /* workspace missing or smaller than the query says         */
    CRANE_HIP_E_LAUNCH = 7,      /* the HIP runtime rejected the launch                      */
    CRANE_HIP_E_ALIGN = 8        /* a pointer or stride breaks the 16-byte row alignment     */
};

/* Human-readable text for a status code (static storage). */
const char* crane_hip_strerror(int code);

/* Fused per-head QK-RMSNorm + RoPE + KV-cache append.
 *
 * qkv       [B, S, (Hq+2*Hkv)*D] merged projection rows (Crane's qkv_proj output,
 *           qwen3/modeling.rs:382-387), row r at qkv + r*qkv_row_stride elements
 * q_norm_w, k_norm_w  [D] RmsNorm weights, or NULL for weight 1 (ignored for ROPE_ONLY)
 * eps       RmsNorm epsilon (config rms_norm_eps)
 * cos, sin  [table_rows, D/2] tables in `dtype`, row p at cos + p*cs_stride elements
 * positions [B] int32, device: token s of sequence b uses table row positions[b]+s;
 *           a token whose row falls outside [0, table_rows) is not written
 * q_out     [B, Hq, S, D] rotated (and normed) queries
 * k_cache, v_cache [B, Hkv, cache_cap, D]: token s of sequence b lands in row
 *           cache_len[b]+s; no other row is touched
 * cache_len [B] int32, device, the rows already valid per sequence (not updated)
 * max_rows  host-side bound: the caller promises cache_len[b] + S <= max_rows
 *           (<= cache_cap), which the launcher checks against cache_cap; the
 *           kernel additionally skips any token whose row would reach cache_cap.
 * Replaces: see the file header. */
int crane_hip_qknorm_rope_append(const void* qkv, int64_t qkv_row_stride,
                                 const void* q_norm_w, const void* k_norm_w, float eps,
                                 int order, const void* cos, const void* sin, int64_t cs_stride,
                                 int64_t table_rows, const int32_t* positions, void* q_out, void* k_cache,
                                 void* v_cache, int64_t cache_cap, const int32_t* cache_len,
                                 int64_t max_rows, int B, int S, int Hq, int Hkv, int D,
                                 int dtype, void* stream);

/* crane_hip_qknorm_rope_append reading the merged projection's f32 split-K
 * partial products instead of its output rows: parts [n_parts, B*S,
 * (Hq+2*Hkv)*D] as crane_gemm_linear_split (crane_gemm.h) writes them,
 * n_parts 2 or 4, and the projection's bias [(Hq+2*Hkv)*D] in `dtype` or NULL.
 * Each row value is T(sum of the splits in split order + bias), the rounding
 * point of the projection's own output (only the f32 summation order
 * differs), then the same per-head arithmetic and cache writes.  For a
 * decode step's qkv_proj, whose split form reads the activations fewer times
 * per weight byte; its reduction costs no launch.  No counterpart in the
 * reference (candle rounds each matmul's output).  Dense cache only. */
int crane_hip_qknorm_rope_append_parts(const float* parts, int n_parts, const void* qkv_bias,
                                       const void* q_norm_w, const void* k_norm_w, float eps, int order,
                                       const void* cos, const void* sin, int64_t cs_stride, int64_t table_rows,
                                       const int32_t* positions, void* q_out, void* k_cache, void* v_cache,
                                       int64_t cache_cap, const int32_t* cache_len, int64_t max_rows, int B, int S,
                                       int Hq, int Hkv, int D, int dtype, void* stream);

/* Query-only QK-norm + RoPE for a layer that shares another layer's K/V:
 * Hunyuan's cross-layer attention (CLA) path, hunyuan_dense/modeling.rs:502-514,
 * which projects q alone, applies rope then query_layernorm, and attends over
 * the anchor layer's cache (already appended for these tokens).  The same
 * per-head arithmetic as crane_hip_qknorm_rope_append's q rows; no cache is
 * read or written.
 *
 * q         [B, S, Hq*D] rows (row r at q + r*q_row_stride elements)
 * q_norm_w  [D] or NULL (weight 1); order as above (Hunyuan: ROPE_THEN_NORM)
 * q_out     [B, Hq, S, D]; the attention launchers then take the anchor's
 *           cache and lengths. */
int crane_hip_qnorm_rope(const void* q, int64_t q_row_stride, const void* q_norm_w, float eps, int order,
                         const void* cos, const void* sin, int64_t cs_stride, int64_t table_rows,
                         const int32_t* positions, void* q_out, int B, int S, int Hq, int D, int dtype,
                         void* stream);

/* RoPE cos/sin tables [max_pos, dim/2] in `dtype`, built on the host CPU into
 * caller-provided HOST memory (upload them once per model).  Bit-identical to
 * Crane's tables:
 *   qwen3/modeling.rs:117-139 (RotaryEmbedding::new: inv_freq = 1.0f32 /
 *   (f32)(base^(2i/dim)) with the power in f64, f32 products p * inv_freq, f32
 *   cosf/sinf) and :857-864 (the tables cast to the model dtype); alpha > 0
 *   gives Hunyuan's NTK-alpha base theta * alpha^(dim/(dim-2))
 *   (hunyuan_dense/modeling.rs:202-219); alpha = 0 leaves theta as the base.
 * Returns CRANE_HIP_E_INVALID for dim odd or above 1024, max_pos < 0, a null
 * table or a non-positive theta. */
int crane_hip_rope_tables(int dim, double theta, double alpha, int64_t max_pos, int dtype, void* cos_out,
                          void* sin_out);

/* The tables of candle-transformers qwen2 (copy at qwen25/qwen2.rs:47-64):
 * inv_freq and the positions are cast to the model dtype before the product,
 * which is rounded to it; cos/sin are computed in f32 and rounded to it.  In
 * bf16 this rounds positions above 256.  In f32 it equals
 * crane_hip_rope_tables(dim, theta, 0, ...). */
int crane_hip_rope_tables_qwen2(int dim, double theta, int64_t max_pos, int dtype, void* cos_out, void* sin_out);

/* Bytes of workspace crane_hip_attn_decode needs for these sizes (max_kv is
 * the largest kv_len the call may see). */
size_t crane_hip_attn_decode_workspace(int B, int Hq, int Hkv, int D, int64_t max_kv, int dtype);

/* Batched split-KV decode attention, one new token per sequence.
 *
 * q        [B, Hq, D] (the decode q_out of the append)
 * k_cache, v_cache [B, Hkv, cache_cap, D]
 * kv_len   [B] int32, device: sequence b attends rows [0, kv_len[b]) (new token
 *          included); 1 <= kv_len[b] <= max_kv <= cache_cap.  A sequence with
 *          kv_len[b] == 0 gets an all-zero output row.
 * scale    softmax scale (1/sqrt(D) in every supported model)
 * score_mode CRANE_HIP_SCORE_GROUPED or CRANE_HIP_SCORE_STANDARD: the candle SDPA
 *          form whose score rounding the call reproduces (see crane_hip_score)
 * out      [B, 1, Hq*D]
 * workspace device scratch of at least crane_hip_attn_decode_workspace(...) bytes,
 *          16-byte aligned, any contents (partial results of the split-KV pass);
 *          calls that overlap in time must not share a workspace.
 * A sequence of at most 256 keys gets candle's softmax_last_dim chain in the
 * model dtype, whatever the other sequences of the batch; longer ones are
 * split over key chunks (256 keys, 512 when max_kv > 12288) whose partial
 * results are merged by their log-sum-exp, so the last bits of a long
 * sequence's output depend on max_kv (the chunk size fixes the f32
 * summation order).
 * Replaces: qwen3/modeling.rs:432-467 and :1118-1200 (see the file header). */
int crane_hip_attn_decode(const void* q, const void* k_cache, const void* v_cache,
                          int64_t cache_cap, const int32_t* kv_len, int64_t max_kv, int B,
                          int Hq, int Hkv, int D, float scale, int score_mode, void* workspace,
                          size_t ws_bytes, void* out, int dtype, void* stream);

/* crane_hip_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference: Crane's candle ops
 * allocate their outputs and temporaries per call.
 * The split-KV partials go in a device array of the library, one per GPU, of
 * crane_hip_attn_decode_noalloc_limit() bytes (32 MiB), held until the process
 * ends; sizes whose crane_hip_attn_decode_workspace(...) exceeds it return
 * CRANE_HIP_E_WORKSPACE.  The call allocates nothing (the array's address is
 * looked up on a device's first call).  Calls that overlap in time on one GPU
 * share the array and race: order them on one stream.  Other arguments and
 * results as crane_hip_attn_decode. */
int crane_hip_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                  int64_t cache_cap, const int32_t* kv_len, int64_t max_kv, int B,
                                  int Hq, int Hkv, int D, float scale, int score_mode, void* out,
                                  int dtype, void* stream);
size_t crane_hip_attn_decode_noalloc_limit(void);

/* Bits of the prefill launchers' `flags` argument.
 *   CAUSAL  -- key j is visible to query i iff j <= start_pos[b]+i
 *              (qwen3/modeling.rs:866-884); without it all start_pos[b]+S keys
 *              are visible.  flags = 0 / 1 keep the meaning of a plain
 *              causal = false / true.
 *   LONG_ROWS_ONE_ROUNDING -- opt-in, bf16 only: query tiles of 128 rows whose
 *              first row sees at least 1024 keys keep candle's first score
 *              rounding only (q@K^T rounded to T, :487) and fold the scale into
 *              the exponent, two VALU instructions fewer per score.  The
 *              second rounding's effect averages out over that many keys, but
 *              the bits of a row then depend on where its 128-row tile starts.
 *              Without the flag every score follows both of candle's
 *              roundings. */
#define CRANE_HIP_PREFILL_CAUSAL 1
#define CRANE_HIP_PREFILL_LONG_ROWS_ONE_ROUNDING 2

/* Causal (or full) GQA prefill attention over the cache.
 *
 * q        [B, Hq, S, D] (the prefill q_out of the append)
 * k_cache, v_cache [B, Hkv, cache_cap, D], holding rows [0, start_pos[b]+S)
 * start_pos [B] int32, device: the rows cached before this chunk; query i of
 *          sequence b sits at position start_pos[b]+i
 * max_start host-side bound: start_pos[b] <= max_start and max_start + S <= cache_cap
 * flags    CRANE_HIP_PREFILL_* bits (above); any other bit is CRANE_HIP_E_INVALID
 * out      [B, S, Hq*D] (qwen3/modeling.rs:497-500)
 * bf16 scores follow candle's two roundings ((q@K^T) rounded to T, then
 * * scale rounded to T, :487-488) unless LONG_ROWS_ONE_ROUNDING is set; rows
 * whose keys all lie in the first 64 get candle's softmax chain in T exactly,
 * other rows an online softmax in f32 over bf16 p.
 * Replaces: qwen3/modeling.rs:469-502 (see the file header). */
int crane_hip_attn_prefill(const void* q, const void* k_cache, const void* v_cache,
                           int64_t cache_cap, const int32_t* start_pos, int64_t max_start,
                           int B, int S, int Hq, int Hkv, int D, float scale, int flags,
                           void* out, int dtype, void* stream);

/* ---- Paged KV cache ------------------------------------------------------
 *
 * The same three operations over a paged cache: K and V pools
 * [n_pages, Hkv, page_rows, D] (rows of D contiguous, as in Crane's layout)
 * and a block table (int32, device) of `table_stride` page ids per sequence.
 * Row j of sequence b is row j % page_rows of page
 * block_table[b * table_stride + j / page_rows]; a sequence holds at most
 * table_stride * page_rows rows.  page_rows is a positive multiple of
 * CRANE_HIP_PAGE_ALIGN (a decode work item then never straddles a page).  A
 * page id outside [0, n_pages) is never dereferenced: its rows read as zeros
 * and are not written.
 *
 * Sequences keep their rows where they were appended, so batched decode reads
 * every sequence in place, a batch is a set of table rows, and growth is a new
 * page id.  This replaces the per-round KV copies of Crane's batched decode
 * (setup_batch_decode + pad_and_stack_kv_caches, qwen3/modeling.rs:973-1030,
 * 1141-1200; extract_batch_kv :1066-1102) and the reallocation copy of
 * update_kv_cache when a buffer is full (:333-355).  Arguments not described
 * here mean what they mean for the dense launchers above; the decode workspace
 * is sized by crane_hip_attn_decode_workspace. */
#define CRANE_HIP_PAGE_ALIGN 256

/* crane_hip_qknorm_rope_append into the pools: token s of sequence b lands in
 * row cache_len[b]+s of that sequence (a row past its capacity or on an
 * invalid page is not written). */
int crane_hip_qknorm_rope_append_paged(const void* qkv, int64_t qkv_row_stride,
                                       const void* q_norm_w, const void* k_norm_w, float eps,
                                       int order, const void* cos, const void* sin, int64_t cs_stride,
                                       int64_t table_rows, const int32_t* positions, void* q_out,
                                       void* k_pool, void* v_pool, int64_t n_pages, int page_rows,
                                       const int32_t* block_table, int64_t table_stride,
                                       const int32_t* cache_len, int B, int S, int Hq, int Hkv, int D,
                                       int dtype, void* stream);

/* crane_hip_attn_decode over the pools (max_kv <= table_stride * page_rows). */
int crane_hip_attn_decode_paged(const void* q, const void* k_pool, const void* v_pool,
                                int64_t n_pages, int page_rows, const int32_t* block_table,
                                int64_t table_stride, const int32_t* kv_len, int64_t max_kv, int B,
                                int Hq, int Hkv, int D, float scale, int score_mode, void* workspace,
                                size_t ws_bytes, void* out, int dtype, void* stream);

/* crane_hip_attn_prefill over the pools (max_start + S <= table_stride * page_rows). */
int crane_hip_attn_prefill_paged(const void* q, const void* k_pool, const void* v_pool,
                                 int64_t n_pages, int page_rows, const int32_t* block_table,
                                 int64_t table_stride, const int32_t* start_pos, int64_t max_start,
                                 int B, int S, int Hq, int Hkv, int D, float scale, int flags,
                                 void* out, int dtype, void* stream);

/* Library and kernel-build identification, e.g. "crane_hip 1 gfx950". */
const char* crane_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif /* CRANE_HIP_H */
