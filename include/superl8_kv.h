/*
 * superl8_kv.h -- C ABI of the MI355X (gfx950) quantized paged KV-cache path.
 *
 * Drop-in boundary for the kernels that jajmangold/superl8-serve reaches through
 * the external `superl8` Python package.  Every entry point takes plain device
 * pointers, element strides and sizes, runs on the HIP stream passed in
 * `stream` (a hipStream_t; NULL = the default stream), never synchronizes,
 * never allocates device memory, and returns an S8KV_* status code.  On a
 * non-zero status `s8kv_last_error()` returns a message for the calling thread.
 *
 * Cache layout (superl8serve/engine/kv_cache.py:484-512), one layer per call:
 *   k_cache, v_cache : int8    [num_blocks, num_kv_heads, block_size, head_dim]
 *   k_scale, v_scale : float32 [num_blocks, num_kv_heads, block_size]
 *   v_packed (k8v3)  : int32   [num_blocks, num_kv_heads, block_size, head_dim*3/32]
 *   v_norm   (k8v3)  : float32 [num_blocks, num_kv_heads, block_size, head_dim/128]
 *   v_codebook(k8v3) : float32 [8]
 * A flat slot s addresses block s / block_size, offset s % block_size
 * (kv_cache.py:570-585).  block_size must be a power of two >= 4 and
 * head_dim one of 32, 64, 128, 256 (k8v3: 128 or 256, lloyd_block 128).
 */
#ifndef SUPERL8_KV_H_
#define SUPERL8_KV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S8KV_OK 0
#define S8KV_ERR_INVALID (-1)     /* bad shape, stride, size or pointer */
#define S8KV_ERR_UNSUPPORTED (-2) /* valid but not implemented (e.g. head_dim 96) */
#define S8KV_ERR_LAUNCH (-3)      /* the HIP runtime rejected a launch */
#define S8KV_ERR_WORKSPACE (-4)   /* workspace missing or too small */

/* Library version (major*10000 + minor*100 + patch). */
int s8kv_version(void);

/* Message for the last non-zero status returned on this thread. */
const char* s8kv_last_error(void);

/*
 * Paged int8 append: quantize-on-write of fp16 K/V into the int8 cache.
 * Replaces superl8.quantize_kv_write_paged(k, v, k_cache, k_scale, v_cache,
 * v_scale, slot_mapping) called at kv_cache.py:1073-1081 (prefill / varlen),
 * kv_cache.py:1108-1116 (decode / verify) and kv_cache.py:288-296 (compaction).
 *
 * k, v: fp16 [num_tokens, num_kv_heads, head_dim]; element strides for the
 * token and head axes, head_dim contiguous.  K is Hadamard-rotated then
 * per-(token, head) symmetric RTN int8 with an fp32 scale (kv_cache.py:587-604);
 * V is RTN without rotation.  Tokens whose slot is negative are skipped.
 */
int s8kv_append_int8(const void* k, const void* v, int64_t num_tokens, int num_kv_heads, int head_dim,
                     int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h,
                     const int32_t* slot_mapping, int8_t* k_cache, float* k_scale, int8_t* v_cache,
                     float* v_scale, int64_t num_blocks, int block_size, void* stream);

/*
 * Paged K8V3 append: K as s8kv_append_int8; V through the 3-bit Lloyd-Max codec
 * (per-128-element L2 norm, nearest codebook entry, bit-plane packing).
 * Replaces the two-step Python write PagedKVCache._write_k_int8 +
 * _write_v_lloydmax3 (kv_cache.py:587-626) reached from write_prefill_varlen /
 * write_decode_static (kv_cache.py:1068-1071, 1103-1106).
 */
int s8kv_append_k8v3(const void* k, const void* v, int64_t num_tokens, int num_kv_heads, int head_dim,
                     int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h,
                     const int32_t* slot_mapping, int8_t* k_cache, float* k_scale, int32_t* v_packed,
                     float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                     int block_size, void* stream);

/*
 * Bytes of scratch device memory the decode entry points need for this
 * geometry on the current device (partial softmax states of rows split across
 * workgroups, and one 8-byte arrival counter per (KV head, row)).  Depends
 * only on its arguments and the device's compute-unit count, so a caller can
 * size the workspace once per graph bucket; max_context_len does not change
 * it.  The workspace must be 8-byte aligned; it needs no initialisation (each
 * launch tags its counters, and the last arrival of a row clears its word),
 * and calls that overlap on one workspace race.
 */
int64_t s8kv_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                   int max_context_len);

/*
 * Ragged-batch GQA decode attention over the int8 paged cache.
 * Replaces superl8.attn_paged_decode_cached(q, k_cache, k_scale, v_cache,
 * v_scale, block_table, context_lens, block_size, *, max_context_len, scale)
 * called at kv_cache.py:1190-1201 (and S times per chain-verify step,
 * gqa_attention.py:259-291).
 *
 * q: fp16 [batch, num_q_heads, head_dim] with element strides q_stride_b,
 * q_stride_h (head_dim contiguous; a [B,Hq,1,D] transpose view qualifies).
 * block_table: int32 [batch, >= ceil(max_context_len/block_size)] with row
 * stride block_table_stride; row b is read only for its first
 * ceil(context_lens[b]/block_size) entries.  context_lens: int32 [batch].
 * max_context_len >= max(context_lens) bounds the block-table width read; a
 * row whose context_lens entry exceeds it is truncated to max_context_len
 * tokens.  A row with context length 0 yields zeros.  max_context_len < 2^28.
 * out: fp16 [batch, num_q_heads, head_dim] contiguous.
 * Row b, head h attends tokens [0, context_lens[b]) of KV head
 * h / (num_q_heads / num_kv_heads) with softmax scale `scale`, applying the
 * Hadamard rotation to q (K is stored rotated).
 */
int s8kv_decode_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                     int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache, const float* k_scale,
                     const int8_t* v_cache, const float* v_scale, int64_t num_blocks, int block_size,
                     const int32_t* block_table, int64_t block_table_stride, const int32_t* context_lens,
                     int max_context_len, float scale, void* out, void* workspace, int64_t workspace_bytes,
                     void* stream);

/*
 * One decode step of a layer in one launch: append, then attend.  Row b's new
 * token (k_new / v_new [batch][num_kv_heads][head_dim] fp16, element strides
 * given, unit stride on head_dim) is quantized exactly as s8kv_append_int8
 * does and written at position context_lens[b] - 1 of row b's block table;
 * the attention then covers positions 0 .. context_lens[b] - 1 as
 * s8kv_decode_int8 does.  Replaces the pair quantize_kv_write_paged
 * (write_decode_static, kv_cache.py:1103-1116) + attn_paged_decode_cached
 * (decode_attn_static, kv_cache.py:1190-1201) when the appended slots are the
 * rows' next positions, which is how the reference's decode step computes
 * them (gqa_attention.py:174-190; kv_cache.py:1083-1093 and 1129-1146 write
 * at lengths[i] and attend lengths[i] + 1 tokens).  Rows with context_lens[b] == 0 or
 * > max_context_len append nothing.  The block holding a row's new token must
 * not be read by another row of the same call.  Other arguments and the
 * workspace as s8kv_decode_int8.
 */
int s8kv_decode_append_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_new_stride_b,
                            int64_t k_new_stride_h, const void* v_new, int64_t v_new_stride_b,
                            int64_t v_new_stride_h, int8_t* k_cache, float* k_scale, int8_t* v_cache, float* v_scale,
                            int64_t num_blocks, int block_size, const int32_t* block_table,
                            int64_t block_table_stride, const int32_t* context_lens, int max_context_len, float scale,
                            void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Allocation-free form of s8kv_decode_append_int8.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels, cache bytes and output as s8kv_decode_append_int8,
 * with no workspace argument: the workspace is a static device array of
 * S8KV_NOALLOC_SCRATCH_BYTES bytes in the library, one copy per GPU, held
 * until the process ends; its device address is looked up once per device on
 * the first call with that device current (the stream and the tensors must be
 * on the current device).  A geometry whose workspace
 * (s8kv_decode_workspace_size) exceeds it is rejected with
 * S8KV_ERR_WORKSPACE.  The scratch needs no clearing (each launch tags its
 * counters, and a row's last arrival zeroes its word), but every call on one
 * GPU shares it: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialized by the caller.  Calls no allocating routine.
 */
#define S8KV_NOALLOC_SCRATCH_BYTES (32ll << 20)
int s8kv_decode_append_int8_noalloc(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                    int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                                    int64_t k_new_stride_b, int64_t k_new_stride_h, const void* v_new,
                                    int64_t v_new_stride_b, int64_t v_new_stride_h, int8_t* k_cache, float* k_scale,
                                    int8_t* v_cache, float* v_scale, int64_t num_blocks, int block_size,
                                    const int32_t* block_table, int64_t block_table_stride,
                                    const int32_t* context_lens, int max_context_len, float scale, void* out,
                                    void* stream);

/*
 * s8kv_decode_append_int8 for the K8V3 layout: the new token is written as
 * s8kv_append_k8v3 writes it (int8 K, 3-bit Lloyd-Max V words and per-128
 * block norms) at position context_lens[b] - 1, then the row attends as
 * s8kv_decode_k8v3 does.  Replaces the reference's K8V3 write
 * (_write_k_int8 + _write_v_lloydmax3, kv_cache.py:587-626) followed by
 * attn_paged_decode_k8v3 (kv_cache.py:1167-1182).  head_dim 128 or 256,
 * lloyd_block 128.
 */
int s8kv_decode_append_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_new_stride_b,
                            int64_t k_new_stride_h, const void* v_new, int64_t v_new_stride_b,
                            int64_t v_new_stride_h, int8_t* k_cache, float* k_scale, int32_t* v_packed,
                            float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                            int block_size, const int32_t* block_table, int64_t block_table_stride,
                            const int32_t* context_lens, int max_context_len, float scale, void* out,
                            void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Per-step slice plan of the decode launches.  No counterpart in the
 * reference (its decode op locates its work per call); it serves the step
 * the reference runs as one decode call per layer with the same block_table
 * and context_lens (ModelRunner's decode step, gqa_attention.py:174-190).
 * s8kv_decode_plan computes, from block_table and context_lens only, the
 * split of the token stream over the decode workgroups and the storage rows
 * of each workgroup's first tiles -- what every decode launch of the step
 * would otherwise compute in its prologue -- into `plan` (device memory,
 * 4-byte aligned, at least s8kv_decode_plan_size(num_kv_heads) bytes).
 * layout: 0 int8, 1 K8V3; fused: 1 for the s8kv_decode_append_* launches.
 * The other arguments are those of the decode launches the plan is for.
 * Stream-ordered, no host synchronization, capturable.
 */
int64_t s8kv_decode_plan_size(int num_kv_heads);
int s8kv_decode_plan(int batch, int num_q_heads, int num_kv_heads, int head_dim, int layout, int fused,
                     int64_t num_blocks, int block_size, const int32_t* block_table, int64_t block_table_stride,
                     const int32_t* context_lens, int max_context_len, void* plan, int64_t plan_bytes, void* stream);

/*
 * s8kv_decode_plan with slice bounds that follow the measured workgroup
 * times.  No counterpart in the reference; same callers as s8kv_decode_plan.
 * The planned decode launches reading an adaptive plan record each
 * workgroup's start and end time in the plan buffer, so `plan` is written by
 * them (launches running at the same time just overwrite each other's
 * times).  The next s8kv_decode_plan_adaptive call into the same buffer
 * moves every workgroup column's share of the token stream a quarter of the
 * way towards the share that equalizes finish times (at most 25% per step).
 * It falls back to the fixed split when the buffer holds no earlier adaptive
 * plan of this geometry, the stream length moved by more than a sixteenth,
 * or some workgroup's times are missing.  Any buffer contents yield a valid
 * split.  Cache bytes are the same as with the fixed split; outputs differ
 * only by the rounding of combining rows split across workgroups.
 */
int s8kv_decode_plan_adaptive(int batch, int num_q_heads, int num_kv_heads, int head_dim, int layout, int fused,
                              int64_t num_blocks, int block_size, const int32_t* block_table,
                              int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                              void* plan, int64_t plan_bytes, void* stream);

/*
 * s8kv_decode_append_int8 / s8kv_decode_append_k8v3 reading a plan made by
 * s8kv_decode_plan for the same geometry and the same block_table and
 * context_lens buffers, whose contents must not have changed since: the
 * launch then issues its first K/V loads at once.  Same cache bytes and
 * outputs as the unplanned calls (the plan holds exactly what their prologue
 * computes).  A plan whose header names another geometry or other buffers is
 * ignored (the launch locates its work itself).  plan_bytes: the plan
 * buffer's size, at least s8kv_decode_plan_size(num_kv_heads) (smaller:
 * S8KV_ERR_INVALID).  Replace the same reference calls as the unplanned
 * forms.  A plan made by s8kv_decode_plan_adaptive is also written: each
 * workgroup records its start and end time in it.
 */
int s8kv_decode_append_int8_planned(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                    int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                                    int64_t k_new_stride_b, int64_t k_new_stride_h, const void* v_new,
                                    int64_t v_new_stride_b, int64_t v_new_stride_h, int8_t* k_cache, float* k_scale,
                                    int8_t* v_cache, float* v_scale, int64_t num_blocks, int block_size,
                                    const int32_t* block_table, int64_t block_table_stride,
                                    const int32_t* context_lens, int max_context_len, float scale, void* out,
                                    void* workspace, int64_t workspace_bytes, void* stream, const void* plan,
                                    int64_t plan_bytes);
int s8kv_decode_append_k8v3_planned(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                    int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                                    int64_t k_new_stride_b, int64_t k_new_stride_h, const void* v_new,
                                    int64_t v_new_stride_b, int64_t v_new_stride_h, int8_t* k_cache, float* k_scale,
                                    int32_t* v_packed, float* v_norm, const float* v_codebook, int lloyd_block,
                                    int64_t num_blocks, int block_size, const int32_t* block_table,
                                    int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                                    float scale, void* out, void* workspace, int64_t workspace_bytes, void* stream,
                                    const void* plan, int64_t plan_bytes);

/*
 * Decode attention over the K8V3 cache (int8 K, 3-bit Lloyd-Max V dequantized
 * in-kernel).  Replaces superl8.attn_paged_decode_k8v3(q, k_cache, k_scale,
 * v_packed, v_norm, v_codebook, block_table, context_lens, block_size, *,
 * max_context_len, scale) called at kv_cache.py:1170-1182.  Arguments as
 * s8kv_decode_int8; head_dim 128 or 256 and lloyd_block 128 (the reference's
 * own gate, kv_cache.py:691-701).
 */
int s8kv_decode_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                     int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache, const float* k_scale,
                     const int32_t* v_packed, const float* v_norm, const float* v_codebook, int lloyd_block,
                     int64_t num_blocks, int block_size, const int32_t* block_table,
                     int64_t block_table_stride, const int32_t* context_lens, int max_context_len, float scale,
                     void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Sliding-window decode: s8kv_decode_int8 / s8kv_decode_k8v3 where row b
 * attends only its last `window` tokens, positions
 * [max(0, L - window), L) for L = min(context_lens[b], max_context_len).
 * The reference's paged kernels have no window; its sliding-window layers
 * read the window back dense (read_dense(..., window=window_left),
 * kv_cache.py:1233-1299) and run a dense decode per row
 * (gqa_attention.py:191-196).  window >= 1; other arguments, the workspace
 * and head_dim support as the unwindowed entry points.
 */
int s8kv_decode_window_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache, const float* k_scale,
                            const int8_t* v_cache, const float* v_scale, int64_t num_blocks, int block_size,
                            const int32_t* block_table, int64_t block_table_stride, const int32_t* context_lens,
                            int max_context_len, int window, float scale, void* out, void* workspace,
                            int64_t workspace_bytes, void* stream);
int s8kv_decode_window_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache, const float* k_scale,
                            const int32_t* v_packed, const float* v_norm, const float* v_codebook, int lloyd_block,
                            int64_t num_blocks, int block_size, const int32_t* block_table,
                            int64_t block_table_stride, const int32_t* context_lens, int max_context_len, int window,
                            float scale, void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Multi-query verify attention over the int8 paged cache: tree verify and
 * chunked prefill.  No single reference op: it computes what the reference
 * gets from S sequential paged decodes in chain verify
 * (gqa_attention.py:217-292, one decode per draft with context L+t+1) and from
 * read_dense + attn_int8_fwd(causal=True) with bottom-right alignment in
 * chunked prefill (gqa_attention.py:105-129, gated_gqa_attention.py:153-191);
 * for a tree it generalizes the chain to an ancestor mask.
 *
 * q: fp16 [batch, num_q_heads, max_queries, head_dim] with element strides
 * q_stride_b, q_stride_h, q_stride_s (head_dim contiguous).  Row b has
 * prefix_lens[b] prefix keys followed by query_lens[b] draft keys (or
 * max_queries when query_lens is NULL), already appended to the cache at
 * positions prefix_lens[b] .. prefix_lens[b]+n-1.  Query s of row b attends
 * every prefix key plus draft key i when i <= s (tree_mask NULL: chain /
 * causal chunk) or when bit i of tree_mask[b*max_queries + s] is set (tree;
 * at most 64 drafts).  Keys at positions >= max_context_len are not read.
 * out: fp16 [batch, num_q_heads, max_queries, head_dim] contiguous; queries
 * s >= query_lens[b] produce zeros.  head_dim 64, 128 or 256.
 *
 * workspace (16-byte aligned, s8kv_verify_workspace_size bytes) lets a call
 * with fewer (sequence, KV head, query block) units than the GPU keeps
 * resident split each unit's keys across workgroups and combine their
 * partials in a second kernel on the same stream (NULL or smaller: no split,
 * a slower call); a call whose units read more than 2^20 keys must split
 * (that bounds the rounding of one workgroup's fp32 sums), and without the
 * workspace it fails with S8KV_ERR_WORKSPACE.  Calls that overlap on one
 * workspace race.  The size covers both layouts (s8kv_verify_int8 and
 * s8kv_verify_k8v3 group query rows differently).
 */
int64_t s8kv_verify_workspace_size(int batch, int num_q_heads, int num_kv_heads, int head_dim, int max_queries,
                                   int max_context_len);

/*
 * Diagnostics (no counterpart in the reference): force the verify's key
 * split to `splits` workgroups per unit (0 restores the per-call plan).
 * Results are the same up to the fp32 rounding of the combined partials.
 */
int s8kv_verify_set_splits(int splits);
int s8kv_verify_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim, int max_queries,
                     int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s, const int8_t* k_cache,
                     const float* k_scale, const int8_t* v_cache, const float* v_scale, int64_t num_blocks,
                     int block_size, const int32_t* block_table, int64_t block_table_stride,
                     const int32_t* prefix_lens, const int32_t* query_lens, const int64_t* tree_mask,
                     int max_context_len, float scale, void* out, void* workspace, int64_t workspace_bytes,
                     void* stream);

/*
 * s8kv_verify_int8 over the K8V3 cache (int8 K, 3-bit Lloyd-Max V): the
 * one-launch form of the reference's chain verify on a k8v3 cache, which runs
 * S sequential decodes that dispatch to attn_paged_decode_k8v3
 * (gqa_attention.py:259-277, kv_cache.py:1168-1188), and of its k8v3 chunked
 * prefill (read_dense, kv_cache.py:1233-1299, then attn_int8_fwd).  V is
 * codebook[code] * block norm; v_packed int32 [num_blocks, Hkv, bs, 3*D/32],
 * v_norm fp32 [num_blocks, Hkv, bs, D/128], v_codebook fp32 [8].  Other
 * arguments as s8kv_verify_int8; head_dim 128 or 256 and lloyd_block 128
 * (the reference's own k8v3 gate, kv_cache.py:691-701).
 */
int s8kv_verify_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim, int max_queries,
                     int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s, const int8_t* k_cache,
                     const float* k_scale, const int32_t* v_packed, const float* v_norm, const float* v_codebook,
                     int lloyd_block, int64_t num_blocks, int block_size, const int32_t* block_table,
                     int64_t block_table_stride, const int32_t* prefix_lens, const int32_t* query_lens,
                     const int64_t* tree_mask, int max_context_len, float scale, void* out, void* workspace,
                     int64_t workspace_bytes, void* stream);

/*
 * Verify attention of a sliding-window layer: as s8kv_verify_int8 /
 * s8kv_verify_k8v3, but of the prefix only the last `window` keys,
 * [max(0, prefix_lens[b] - window), prefix_lens[b]), are visible (drafts as
 * before).  The reference reads that prefix window back dense and appends the
 * drafts' fresh fp16 K / V (gqa_attention.py:298-314, read_dense at
 * kv_cache.py:1233-1299): pass them as k_draft (fp32, already rotated:
 * s8kv_rotate_rows of the fp16 K) and v_draft (fp16), each
 * [batch][max_queries][num_kv_heads][head_dim] at element strides (per row,
 * draft, head; rows 16-byte aligned), and draft i of row b is attended with
 * those values instead of its cache row (K carried as fp16 hi + lo).  k_draft NULL: the drafts are read
 * from the cache, as the unwindowed verify reads them.  window >= 1.
 */
int s8kv_verify_window_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                            const int8_t* k_cache, const float* k_scale, const int8_t* v_cache, const float* v_scale,
                            int64_t num_blocks, int block_size, const int32_t* block_table,
                            int64_t block_table_stride, const int32_t* prefix_lens, const int32_t* query_lens,
                            const int64_t* tree_mask, int max_context_len, int window, const void* k_draft,
                            int64_t kd_stride_b, int64_t kd_stride_s, int64_t kd_stride_h, const void* v_draft,
                            int64_t vd_stride_b, int64_t vd_stride_s, int64_t vd_stride_h, float scale, void* out,
                            void* workspace, int64_t workspace_bytes, void* stream);
int s8kv_verify_window_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                            const int8_t* k_cache, const float* k_scale, const int32_t* v_packed,
                            const float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                            int block_size, const int32_t* block_table, int64_t block_table_stride,
                            const int32_t* prefix_lens, const int32_t* query_lens, const int64_t* tree_mask,
                            int max_context_len, int window, const void* k_draft, int64_t kd_stride_b,
                            int64_t kd_stride_s, int64_t kd_stride_h, const void* v_draft, int64_t vd_stride_b,
                            int64_t vd_stride_s, int64_t vd_stride_h, float scale, void* out, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * Prefill attention over fresh fp16 K / V (not the cache), varlen batched:
 * the role of superl8.attn_int8_varlen (gqa_attention.py:81-104) and of
 * attn_int8_fwd over fresh K / V (gqa_attention.py:124-128).  Sequence b's
 * queries are tokens cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1 of q
 * [tokens, num_q_heads, head_dim] and its keys tokens cu_seqlens_k[b] .. of
 * k, v [tokens, num_kv_heads, head_dim] (element strides per token and head,
 * head_dim contiguous; K and V rows 16-byte aligned).  causal: query s sees
 * keys j <= s + nk - nq (bottom-right aligned; none when that is negative),
 * else all nk keys; window_left >= 1 (causal only) also hides keys
 * j <= s + nk - nq - window_left, so each query sees its last window_left
 * keys, itself included (the window the reference's sliding-window decode
 * attends: gqa_attention.py:150-154, read_dense(window=) at
 * kv_cache.py:1233-1299); -1 for none, 0 is rejected.
 * out [tokens_q, num_q_heads, head_dim] with strides
 * o_stride_t, o_stride_h; only the sequences' own query tokens are written.
 * The causal diagonal comes from each sequence's own counts.  max_seqlen_q
 * sizes the grid and must be >= every sequence's query count (queries past it
 * are not computed); max_seqlen_k is informational.  cu_seqlens must be
 * non-decreasing and within the q / k / v token counts: K, V and out are
 * addressed from them without further bounds.
 * head_dim 64, 128 or 256; at most 16 q heads per KV head.
 */
int s8kv_attn_varlen_f16(const void* q, const void* k, const void* v, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                         int max_seqlen_q, int max_seqlen_k, int64_t q_stride_t, int64_t q_stride_h,
                         int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h, int causal,
                         int window_left, float scale, void* out, int64_t o_stride_t, int64_t o_stride_h,
                         void* stream);

/*
 * Row codecs behind the helpers the reference's cache code calls on the
 * `superl8` module.  Rows are head_dim contiguous elements at a uniform row
 * stride (in elements); outputs are contiguous [num_rows][...].  Each gives
 * the bytes the append kernels write for the same row.
 *
 * s8kv_rotate_rows: out = rotate_last(x), the Hadamard rotation
 * superl8.quant.rotation.rotate_last called at kv_cache.py:594-597 (K side of
 * the k8v3 write), kv_cache.py:1272 and 1297 (read_dense un-rotating K):
 * fp32 Walsh-Hadamard transform, one fp32 multiply by fp32(1/sqrt(head_dim)),
 * one rounding to the element type.  dtype: 0 fp16, 1 bf16, 2 fp32 (in and
 * out).  head_dim 32, 64, 128 or 256.
 */
int s8kv_rotate_rows(const void* x, int64_t num_rows, int head_dim, int64_t x_row_stride, int dtype, void* out,
                     int64_t out_row_stride, void* stream);

/*
 * Per-row symmetric RTN int8 of fp16 rows: superl8.quantize_i8_rowwise called
 * at kv_cache.py:601 on rotate_last(K) (rotate = 0), and the same after the
 * rotation in one pass (rotate = 1, the K side of s8kv_append_int8 and of
 * superl8.quantize_kv_cache, kv_cache.py:1231).  q int8 [num_rows][head_dim],
 * scale fp32 [num_rows] (absmax / 127; 0 for an all-zero row).
 */
int s8kv_quantize_rows_int8(const void* x, int64_t num_rows, int head_dim, int64_t x_row_stride, int rotate,
                            int8_t* q, float* scale, void* stream);

/*
 * 3-bit Lloyd-Max V codec of fp16 rows: superl8.quant.lloydmax.quantize_lloydmax
 * (bits 3, block_size 128, last dim) called at kv_cache.py:613-620.  codes uint8
 * [num_rows][head_dim] (0..7), norms fp32 [num_rows][head_dim/128];
 * codebook fp32 [8].  head_dim 128 or 256.
 */
int s8kv_quantize_rows_lloydmax3(const void* v, int64_t num_rows, int head_dim, int64_t v_row_stride,
                                 const float* codebook, uint8_t* codes, float* norms, void* stream);

/*
 * Bit-plane packing of 3-bit codes and its inverse:
 * superl8.quant.lloydmax.pack_indices_lowbit(codes, 3) at kv_cache.py:623 and
 * unpack_indices_lowbit(packed, 3, head_dim) at kv_cache.py:662 and 1285.
 * codes uint8 [num_rows][head_dim] (taken modulo 8), words int32
 * [num_rows][head_dim*3/32]: word 3g+b holds bit b of the codes of elements
 * 32g .. 32g+31, element 32g+i at bit i (the cache's v_packed layout).
 */
int s8kv_pack_codes3(const uint8_t* codes, int64_t num_rows, int head_dim, int32_t* words, void* stream);
int s8kv_unpack_codes3(const int32_t* words, int64_t num_rows, int head_dim, uint8_t* codes, void* stream);

/*
 * SnapKV scores for prompt-time eviction: score[t] = mean over q heads h of
 * softmax_t(scale * q_h . K_t) over a sequence's `length` keys, the quantity
 * KVEviction.snapkv_selection ranks (kv_cache.py:124-166; GQA: q head h reads
 * KV head h / (num_q_heads / num_kv_heads)).  q: [num_q_heads][head_dim] rows
 * at q_stride elements, fp16 (q_is_f32 = 0) or fp32.  scores fp32 [length].
 * Workspace: s8kv_snapkv_workspace_size bytes (the logits and per-head
 * softmax statistics), 4-byte aligned.
 *
 * _paged: K is the sequence's int8 K in the paged cache (block ids in order
 * at block_row, >= ceil(length / block_size) of them), dequantized exactly
 * (k_i8 * k_scale, un-rotated by rotating q) -- the reference has no paged
 * form; it takes the caller's dense K.  _dense: K fp16 / fp32
 * [num_kv_heads][length][head_dim] with element strides (the reference's
 * k_full).  head_dim 32, 64, 128 or 256; at most 64 q heads per KV head.
 */
int64_t s8kv_snapkv_workspace_size(int num_q_heads, int length);
int s8kv_snapkv_scores_paged(const void* q, int q_is_f32, int64_t q_stride, int num_q_heads, int num_kv_heads,
                             int head_dim, const int8_t* k_cache, const float* k_scale, int64_t num_blocks,
                             int block_size, const int32_t* block_row, int length, float scale, float* scores,
                             void* workspace, int64_t workspace_bytes, void* stream);
int s8kv_snapkv_scores_dense(const void* q, int q_is_f32, int64_t q_stride, int num_q_heads, int num_kv_heads,
                             int head_dim, const void* k, int k_is_f32, int64_t k_stride_h, int64_t k_stride_t,
                             int length, float scale, float* scores, void* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * Keep-list compaction: for each j < num_tokens, every (layer, tensor, KV
 * head) row at flat slot src_slots[j] is copied to flat slot dst_slots[j],
 * byte for byte (tensor i: rows of row_bytes[i] bytes in the cache layout
 * [layer][block][head][offset], layer_stride_bytes[i] apart; up to 8 tensors:
 * k_cache, k_scale, v_cache, v_scale or v_packed, v_norm).  Replaces the
 * dequantize -> un-rotate -> requantize loop of KVEviction.compact
 * (kv_cache.py:249-296), which is lossy; slots outside
 * [0, num_blocks * block_size) move nothing.  Source and destination slots
 * must be disjoint.  src_slots, dst_slots: device int32 [num_tokens].
 */
int s8kv_gather_slots(int num_tensors, void* const* tensor_ptrs, const int64_t* row_bytes,
                      const int64_t* layer_stride_bytes, int num_layers, int num_kv_heads, int64_t num_blocks,
                      int block_size, const int32_t* src_slots, const int32_t* dst_slots, int num_tokens,
                      void* stream);

/*
 * Kernel timing (diagnostics; no counterpart in the reference).  Between
 * s8kv_timing_begin() and s8kv_timing_end(), every decode call made outside
 * graph capture launches its kernel with HIP events stamped with the
 * kernel's start and end; s8kv_timing_end() waits for them and returns the
 * number of decode calls and the summed kernel durations (ms).  merge_ms is
 * always 0: rows split across workgroups are combined inside the kernel.
 * Used by the benchmark to time the attention kernel on its own stream.
 */
int s8kv_timing_begin(void);
int s8kv_timing_end(int* launches, double* decode_ms, double* merge_ms);

/*
 * Read-ceiling probes (diagnostics; no counterpart in the reference).  They
 * read without computing, to bound what a kernel reading the same bytes
 * with the same shape can reach; each workgroup writes one checksum word to
 * sink[num_workgroups] so no load is dropped.
 * s8kv_probe_read_tiles: for each entry of tiles (device int32
 * [num_tiles], the first storage row of a 32-token tile inside one block
 * and head, as the decode kernel reads them), the tile's 32 K rows and 32 V
 * rows (int8, head_dim 128) and their fp32 scales; 4-wave workgroups, each
 * taking an equal contiguous share of the list, one tile per wave with the
 * next tile's loads in flight.  num_rows: storage rows of the cache tensors.
 * s8kv_probe_read_linear: `bytes` contiguous bytes (16-byte aligned).
 */
int s8kv_probe_read_tiles(const int8_t* k_cache, const float* k_scale, const int8_t* v_cache, const float* v_scale,
                          int64_t num_rows, int head_dim, const int32_t* tiles, int num_tiles, int num_workgroups,
                          uint32_t* sink, void* stream);
int s8kv_probe_read_linear(const void* buffer, int64_t bytes, int num_workgroups, uint32_t* sink, void* stream);

/*
 * Copy whole physical blocks across every layer of up to 8 cache tensors
 * (copy-on-write of a shared prefix block; compaction of the pool).
 * The reference has no block copy: prefix sharing is refcounted
 * (kv_cache.py:751-755) and compaction re-quantizes token by token
 * (kv_cache.py:199-313).  This entry point is the byte-exact replacement used
 * behind the build's copy-on-write and compaction.
 *
 * tensor_ptrs[i]: base of tensor i, laid out [num_layers][num_blocks][...];
 * block_bytes[i]: bytes of one block of one layer (a multiple of 16);
 * layer_stride_bytes[i]: bytes between consecutive layers.
 * src_blocks, dst_blocks: device int32 [num_pairs]; the two sets must be
 * disjoint.  Copies t[layer][dst[p]] = t[layer][src[p]] for all layers.
 */
int s8kv_copy_blocks(int num_tensors, void* const* tensor_ptrs, const int64_t* block_bytes,
                     const int64_t* layer_stride_bytes, int num_layers, int64_t num_blocks,
                     const int32_t* src_blocks, const int32_t* dst_blocks, int num_pairs, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SUPERL8_KV_H_ */
