/*
 * helix_paged.h -- C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * Drop-in boundary for the reference's paged cache and paged attention
 * (parthpandya5/helix-runtime).  Every entry point takes plain pointers and
 * sizes; device pointers refer to HIP device memory of the cache's device;
 * `stream` is a hipStream_t (NULL selects the null stream).  No exception
 * crosses this boundary: every function returns a helix_status and stores a
 * message retrievable with helix_last_error() on the calling thread.
 *
 * Citations are "reference file:line" of the interface each entry replaces.
 */
#ifndef HELIX_PAGED_H
#define HELIX_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* helix::ErrorCode (include/helix/core/error.hpp:10-17) shifted by one so
 * that zero means success. */
typedef enum helix_status {
  HELIX_OK = 0,
  HELIX_INVALID_ARGUMENT = 1,
  HELIX_OUT_OF_RANGE = 2,
  HELIX_UNSUPPORTED = 3,
  HELIX_RESOURCE_EXHAUSTED = 4,
  HELIX_RUNTIME = 5,
  HELIX_INTERNAL = 6
} helix_status;

typedef void* helix_stream; /* hipStream_t */

/* PagedKvCacheConfig (include/helix/kv_cache/paged.hpp:60-66). */
typedef struct helix_paged_config {
  size_t layers;
  size_t kv_heads;
  size_t head_dimension;
  size_t block_tokens;
  size_t physical_blocks;
} helix_paged_config;

/* PagedKvCacheStats (include/helix/kv_cache/paged.hpp:68-107), 64-bit. */
typedef struct helix_paged_stats {
  uint64_t bytes_reserved, bytes_used, bytes_free, peak_bytes_used;
  uint64_t total_blocks, used_blocks, free_blocks, active_sequence_count;
  uint64_t active_tokens, resident_tokens, allocated_token_slots;
  uint64_t block_reference_count, shared_blocks;
  uint64_t sequence_create_count, sequence_fork_count, append_count, release_count;
  uint64_t block_allocation_count, block_reuse_count;
} helix_paged_stats;

/* PagedSequenceHandle / CudaPagedSequenceHandle
 * (include/helix/kv_cache/paged.hpp:34-58, cuda_paged.hpp:18-42). id 0 is
 * the empty handle. */
typedef struct helix_sequence {
  uint64_t id;
  uint64_t cache_id;
} helix_sequence;

/* Copy-on-write page copy a fork implies (extension; no reference
 * counterpart, docs/KV_CACHE.md:247): tokens == 0 when none. */
typedef struct helix_cow_copy {
  uint32_t from_block;
  uint32_t to_block;
  size_t tokens;
} helix_cow_copy;

typedef struct helix_block_manager helix_block_manager;
typedef struct helix_paged_cache helix_paged_cache;
typedef struct helix_decode_view helix_decode_view;
typedef struct helix_block_table helix_block_table;
typedef struct helix_decode_batch helix_decode_batch;

/* ----------------------------------------------------------- errors ---- */
/* Message of the last failed call on this thread ("" after success). */
const char* helix_last_error(void);
/* helix::error_code_name (include/helix/core/error.hpp:19). */
const char* helix_status_name(int status);

/* ---------------------------------------------- host page bookkeeping ---- */
/* The metadata half of PagedKvCache (src/kv_cache/paged.cpp), usable without
 * a device: FIFO allocation, block tables, reference counts, statistics. */
int helix_block_manager_create(const helix_paged_config* config, helix_block_manager** out);
void helix_block_manager_destroy(helix_block_manager* manager);
/* PagedKvCache::create_sequence (paged.cpp:509-533). */
int helix_block_manager_create_sequence(helix_block_manager* m, helix_sequence* out);
/* PagedKvCache::fork_sequence (paged.cpp:535-620); allow_cow != 0 accepts a
 * non-aligned prefix and reports the page copy the caller must perform. */
int helix_block_manager_fork_sequence(helix_block_manager* m, helix_sequence source,
                                      size_t prefix_tokens, int allow_cow, helix_sequence* out,
                                      helix_cow_copy* copy);
/* Appends `tokens` tokens (paged.cpp:622-719, 721-871); writes each token's
 * physical slot block * block_tokens + offset into slots (may be NULL). */
int helix_block_manager_append(helix_block_manager* m, helix_sequence sequence, size_t tokens,
                               uint64_t* slots);
/* PagedKvCache::release_sequence (paged.cpp:952-1001). */
int helix_block_manager_release_sequence(helix_block_manager* m, helix_sequence sequence);
int helix_block_manager_contains(const helix_block_manager* m, helix_sequence sequence, int* out);
int helix_block_manager_length(const helix_block_manager* m, helix_sequence sequence,
                               size_t* out);
/* PagedKvCache::block_table (paged.cpp:1014-1023): writes min(count,
 * capacity) IDs and the full count. */
int helix_block_manager_block_table(const helix_block_manager* m, helix_sequence sequence,
                                    uint32_t* out, size_t capacity, size_t* count);
int helix_block_manager_stats(const helix_block_manager* m, helix_paged_stats* out);
int helix_block_manager_block_info(const helix_block_manager* m, uint32_t block,
                                   size_t* reference_count, size_t* token_count);
/* Re-derives every invariant (paged.cpp:282-393); HELIX_INTERNAL on failure. */
int helix_block_manager_validate(const helix_block_manager* m);
/* bytes_per_token / block_bytes / token_capacity (paged.cpp:1035-1045). */
int helix_block_manager_geometry(const helix_block_manager* m, size_t* bytes_per_token,
                                 size_t* block_bytes, size_t* token_capacity);

/* ------------------------------------------------------ device cache ---- */
/* CudaPagedKvCache (include/helix/kv_cache/cuda_paged.hpp:91-116, src/kv_cache/
 * cuda_paged.cpp:454-697) plus the CPU cache's fork and bulk append. */
int helix_paged_cache_create(const helix_paged_config* config, int device,
                             helix_paged_cache** out);
/* Page element type (extension; the reference's pages are fp32 only,
 * docs/KV_CACHE.md:531).  bf16 pages hold each appended fp32 value rounded to
 * nearest even (NaN stays NaN); gathers widen them back to fp32 exactly, and
 * attention over a bf16 cache computes in fp32 on the bf16 values, with the
 * step's fp32 tail rows rounded the same way.  Byte statistics count 2-byte
 * elements.  bf16 caches decode in stream mode only (pages_per_split 0), and
 * the pools helix_paged_cache_layer_pools / helix_decode_view_layer_pools
 * return then hold bf16 bits.
 * fp8 pages (HELIX_PAGE_FP8_E4M3) hold OCP FP8 E4M3 codes with one fp32
 * scale for keys and one for values: an element is the code of x / scale
 * rounded to nearest even, saturating at +-448 (NaN stays NaN), and its value
 * is decode(code) * scale.  Gathers return those values; attention computes
 * in fp32 on them, the step's tail and chunk rows rounded the same way; byte
 * statistics count 1-byte elements; same stream-mode rule as bf16, and the
 * pools hold the codes.  helix_paged_cache_create_typed with FP8 uses scales
 * of 1. */
typedef enum helix_page_dtype {
  HELIX_PAGE_F32 = 0,
  HELIX_PAGE_BF16 = 1,
  HELIX_PAGE_FP8_E4M3 = 2
} helix_page_dtype;
int helix_paged_cache_create_typed(const helix_paged_config* config, int device, int page_dtype,
                                   helix_paged_cache** out);
/* fp8 cache with its key and value scales (finite, positive). */
int helix_paged_cache_create_fp8(const helix_paged_config* config, int device, float key_scale,
                                 float value_scale, helix_paged_cache** out);
int helix_paged_cache_page_dtype(helix_paged_cache* cache, int* out);
/* The key and value scales of an fp8 cache (1 and 1 for the other types). */
int helix_paged_cache_fp8_scales(helix_paged_cache* cache, float* key_scale, float* value_scale);
void helix_paged_cache_destroy(helix_paged_cache* cache);
int helix_paged_cache_create_sequence(helix_paged_cache* cache, helix_sequence* out);
/* PagedKvCache::fork_sequence (paged.cpp:535-620); allow_cow != 0 copies a
 * partial last page on the device (extension). */
int helix_paged_cache_fork_sequence(helix_paged_cache* cache, helix_sequence source,
                                    size_t prefix_tokens, int allow_cow, helix_stream stream,
                                    helix_sequence* out);
/* CudaPagedKvCache::append (cuda_paged.cpp:491-611): token_keys/values are
 * device [layers, kv_heads, head_dim]; one kernel, then a stream sync, then
 * the metadata commit. */
int helix_paged_cache_append(helix_paged_cache* cache, helix_sequence sequence,
                             const float* token_keys, const float* token_values,
                             helix_stream stream);
/* PagedKvCache::append_layer_major (paged.cpp:721-871): host arrays of
 * `layers` device pointers, each [kv_heads, tokens, head_dim]. */
int helix_paged_cache_append_layer_major(helix_paged_cache* cache, helix_sequence sequence,
                                         const float* const* layer_keys,
                                         const float* const* layer_values, size_t tokens,
                                         helix_stream stream);
/* CudaPagedKvCache::release_sequence (cuda_paged.cpp:613-643). */
int helix_paged_cache_release_sequence(helix_paged_cache* cache, helix_sequence sequence);
/* PagedKvCache::copy_layer_out (paged.cpp:887-893): device outputs
 * [kv_heads, length, head_dim]; synchronises the stream. */
int helix_paged_cache_copy_layer_out(helix_paged_cache* cache, helix_sequence sequence,
                                     size_t layer, float* keys_out, float* values_out,
                                     helix_stream stream);
/* PagedKvCache::copy_layer_prefix_out (paged.cpp:895-950): outputs
 * [kv_heads, dest_tokens, head_dim], trailing rows untouched. */
int helix_paged_cache_copy_layer_prefix_out(helix_paged_cache* cache, helix_sequence sequence,
                                            size_t layer, size_t expected_length,
                                            float* keys_out, float* values_out,
                                            size_t dest_tokens, helix_stream stream);
int helix_paged_cache_contains(helix_paged_cache* cache, helix_sequence sequence, int* out);
int helix_paged_cache_length(helix_paged_cache* cache, helix_sequence sequence, size_t* out);
int helix_paged_cache_block_table(helix_paged_cache* cache, helix_sequence sequence,
                                  uint32_t* out, size_t capacity, size_t* count);
int helix_paged_cache_stats(helix_paged_cache* cache, helix_paged_stats* out);
/* CudaPagedKvCache::is_healthy (cuda_paged.cpp:656-659). */
int helix_paged_cache_is_healthy(helix_paged_cache* cache, int* out);
int helix_paged_cache_geometry(helix_paged_cache* cache, size_t* bytes_per_token,
                               size_t* block_bytes, size_t* token_capacity);
/* Device pools of one layer, each [physical_blocks, kv_heads, block_tokens,
 * head_dim] (DecodeView::layer_key_blocks / layer_value_blocks). */
int helix_paged_cache_layer_pools(helix_paged_cache* cache, size_t layer, float** key_blocks,
                                  float** value_blocks);

/* CudaPagedKvCache::read_sequence / DecodeView (cuda_paged.cpp:377-452,
 * 645-654).  The view holds the cache mutex until released, from the same
 * thread; append and release block meanwhile. */
int helix_paged_cache_read_sequence(helix_paged_cache* cache, helix_sequence sequence,
                                    helix_decode_view** out);
int helix_decode_view_length(const helix_decode_view* view, size_t* out);
int helix_decode_view_physical_blocks(const helix_decode_view* view, const uint32_t** blocks,
                                      size_t* count);
/* Device copy of the block table (NULL for an empty sequence). */
int helix_decode_view_block_table(const helix_decode_view* view, const uint32_t** device_table);
int helix_decode_view_layer_pools(const helix_decode_view* view, size_t layer,
                                  float** key_blocks, float** value_blocks);
/* DecodeView::poison_after_consumer_failure (cuda_paged.cpp:441-452). */
void helix_decode_view_poison(helix_decode_view* view);
void helix_decode_view_release(helix_decode_view* view);

/* PagedBlockTable (include/helix/kv_cache/cuda_block_table.hpp:16-47,
 * src/kv_cache/cuda_block_table.cpp:22-47): validates every ID against
 * physical_block_count, then uploads synchronously.  Empty tables own no
 * device memory and report a NULL data pointer. */
int helix_block_table_create(const uint32_t* physical_blocks, size_t count,
                             size_t physical_block_count, int device, helix_block_table** out);
const uint32_t* helix_block_table_data(const helix_block_table* table);
size_t helix_block_table_logical_block_count(const helix_block_table* table);
void helix_block_table_destroy(helix_block_table* table);

/* ------------------------------------------- reference-shaped attention ---- */
/* Shapes (the reference's attention::cuda contract, include/helix/attention/
 * cuda_paged.hpp:15-69):
 *   query        [q_heads, queries, key_dim]
 *   key_blocks   [physical_blocks, kv_heads, block_tokens, key_dim]
 *   value_blocks [physical_blocks, kv_heads, block_tokens, value_dim]
 *   block_table  logical_blocks device uint32 IDs
 *   workspace    [q_heads, queries, kv_tokens] -- receives probabilities
 *   output       [q_heads, queries, value_dim]
 * q_heads must be a multiple of kv_heads (the reference requires equality;
 * grouped-query attention is an extension). */

/* paged_score_workspace_bytes (cuda_paged.cu:381-394): validates the
 * history-only geometry and returns q_heads * queries * kv_tokens * 4. */
int helix_paged_score_workspace_bytes(size_t q_heads, size_t queries, size_t kv_heads,
                                      size_t physical_blocks, size_t block_tokens,
                                      size_t logical_blocks, size_t kv_tokens, size_t* out);
/* paged_tail_score_workspace_bytes (cuda_paged.cu:396-418). */
int helix_paged_tail_score_workspace_bytes(size_t q_heads, size_t tail_tokens, size_t kv_heads,
                                           size_t physical_blocks, size_t block_tokens,
                                           size_t logical_blocks, size_t history_tokens,
                                           size_t* out);
/* paged_scaled_dot_product_attention_out (cuda_paged.cu:420-481).  Routes as
 * helix_paged_attention_with_tail_out: one query row on the single-sequence
 * decode kernel, several on the matrix-core prefill kernel (the rows' own
 * page tokens gathered into the stream's scratch as the chunk). */
int helix_paged_attention_out(const float* query, size_t q_heads, size_t queries, size_t key_dim,
                              const float* key_blocks, const float* value_blocks,
                              size_t physical_blocks, size_t kv_heads, size_t block_tokens,
                              size_t value_dim, const uint32_t* block_table,
                              size_t logical_blocks, size_t kv_tokens,
                              size_t query_position_offset, float* output,
                              float* score_workspace, size_t workspace_elements,
                              helix_stream stream);
/* paged_scaled_dot_product_attention_with_tail_out (cuda_paged.cu:483-548):
 * tail_key [kv_heads, tail_tokens, key_dim], tail_value [kv_heads,
 * tail_tokens, value_dim]; query row q sees the history and tail rows 0..q.
 * The reference model's per-layer decode call (src/model/cuda_llama.cpp:
 * 365-367).  The workspace receives the probabilities on every route, as in
 * the reference.  With key_dim = value_dim = 128, 16-token pages, q_heads /
 * kv_heads in {1, 2, 4, 8} and 16-byte aligned rows, a one-token call runs
 * the single-sequence decode kernel (plus a merging launch when a kv head spans
 * several workgroups) and a call with several tail rows (a prefill chunk)
 * runs the exact fp32 matrix-core prefill kernel plus a normalisation
 * launch; both use a device scratch the library keeps per (device, stream),
 * allocated or grown on first use.  Every other call runs the exact scalar
 * kernel. */
int helix_paged_attention_with_tail_out(const float* query, size_t q_heads, size_t tail_tokens,
                                        size_t key_dim, const float* key_blocks,
                                        const float* value_blocks, size_t physical_blocks,
                                        size_t kv_heads, size_t block_tokens, size_t value_dim,
                                        const uint32_t* block_table, size_t logical_blocks,
                                        size_t history_tokens, const float* tail_key,
                                        const float* tail_value, float* output,
                                        float* score_workspace, size_t workspace_elements,
                                        helix_stream stream);
/* The same call with the reference's full workspace contract
 * (cuda_paged.cu:483-548, checked by tests/cuda_attention_test.cpp:443):
 * score_workspace [q_heads, tail_tokens, history + tail] receives the
 * attention probabilities; always the exact scalar kernel (the reference's
 * loop order, no device scratch), whatever the shape. */
int helix_paged_attention_with_tail_probabilities_out(
    const float* query, size_t q_heads, size_t tail_tokens, size_t key_dim,
    const float* key_blocks, const float* value_blocks, size_t physical_blocks, size_t kv_heads,
    size_t block_tokens, size_t value_dim, const uint32_t* block_table, size_t logical_blocks,
    size_t history_tokens, const float* tail_key, const float* tail_value, float* output,
    float* score_workspace, size_t workspace_elements, helix_stream stream);

/* -------------------------------------------- batched decode (extension) ---- */
/* One-token decode for `batch` sequences at once (the reference runs one
 * sequence per call, docs/ATTENTION.md:317):
 *   query [batch, q_heads, head_dim];
 *   key_blocks, value_blocks [physical_blocks, kv_heads, block_tokens, head_dim];
 *   tables [batch, max_blocks] uint32; lengths [batch] int32 history tokens;
 *   tail_key/value [batch, kv_heads, head_dim]; output [batch, q_heads, head_dim].
 * The kernels are built for head_dim 128, 16-token pages and q_heads /
 * kv_heads in {1, 2, 4, 8}; any other geometry returns HELIX_UNSUPPORTED
 * before a launch.  pages_per_split 0 (the default) runs the persistent
 * stream kernel: a fixed grid of wavefronts streams the flat page list of
 * all (sequence, kv head) units, and a merge launch combines the units that
 * span wavefronts.  pages_per_split > 0 instead cuts each sequence's history
 * into splits of that many pages, one wavefront per split (at most 4096
 * splits per sequence), then merges the splits.  The workspace holds the
 * partials (calls that overlap on one workspace race).
 * helix_paged_decode_workspace_init zero-fills a workspace (optional: every
 * call writes the partials it reads). */
int helix_paged_decode_workspace_bytes(size_t batch, size_t q_heads, size_t kv_heads,
                                       size_t max_blocks, size_t pages_per_split, size_t* out);
int helix_paged_decode_workspace_init(void* workspace, size_t workspace_bytes,
                                      helix_stream stream);
int helix_paged_decode_attention(const float* query, size_t batch, size_t q_heads,
                                 size_t kv_heads, size_t head_dim, const float* key_blocks,
                                 const float* value_blocks, size_t physical_blocks,
                                 size_t block_tokens, const uint32_t* tables, size_t max_blocks,
                                 const int32_t* lengths, const float* tail_key,
                                 const float* tail_value, float* output, void* workspace,
                                 size_t workspace_bytes, size_t pages_per_split,
                                 helix_stream stream);
/* helix_paged_decode_attention over bf16 or fp8 E4M3 pools (extension: the
 * reference's pools are fp32 only, docs/KV_CACHE.md:531), for callers that
 * keep reduced-precision pools without a helix_decode_batch.  page_dtype is
 * a helix_page_dtype; key_blocks / value_blocks hold elements of that type
 * (the layout of helix_paged_cache_create_typed / _create_fp8 pools, whose
 * key_scale / value_scale an fp8 call passes: finite and positive; ignored
 * for the other types).  query, tails and output stay fp32.  bf16 and fp8
 * pools take the stream kernel only (pages_per_split 0; otherwise
 * HELIX_UNSUPPORTED); an unknown page_dtype or a bad fp8 scale is
 * HELIX_INVALID_ARGUMENT before any launch.  HELIX_PAGE_F32 is exactly
 * helix_paged_decode_attention. */
int helix_paged_decode_attention_typed(const float* query, size_t batch, size_t q_heads,
                                       size_t kv_heads, size_t head_dim, const void* key_blocks,
                                       const void* value_blocks, size_t physical_blocks,
                                       size_t block_tokens, const uint32_t* tables,
                                       size_t max_blocks, const int32_t* lengths,
                                       const float* tail_key, const float* tail_value,
                                       float* output, void* workspace, size_t workspace_bytes,
                                       size_t pages_per_split, int page_dtype, float key_scale,
                                       float value_scale, helix_stream stream);
/* helix_paged_decode_attention in stream mode without a workspace argument
 * and without any allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The stream kernel's
 * partial results go to a library-owned 16 MiB device array (one per GPU,
 * held until the process ends); batch * kv_heads beyond what it holds
 * (about 6000 (sequence, kv head) units at query groups of 4) returns
 * HELIX_OUT_OF_RANGE.  Every call on one GPU shares that array, so calls
 * that overlap on one GPU (on different streams, or from several threads
 * without ordering) race; calls ordered on one stream do not.  To use it
 * from two streams, order the calls: hipEventRecord(e, s1) after the call on
 * s1, hipStreamWaitEvent(s2, e, 0) before the call on s2.  Nothing in
 * the array needs to start at zero: each call writes every partial it
 * reads.  Same arguments and results as helix_paged_decode_attention_typed
 * with pages_per_split 0 (page_dtype, key_scale and value_scale as there;
 * bf16 and fp8 pools take the same array). */
int helix_paged_decode_attention_noalloc(const float* query, size_t batch, size_t q_heads,
                                         size_t kv_heads, size_t head_dim, const void* key_blocks,
                                         const void* value_blocks, size_t physical_blocks,
                                         size_t block_tokens, const uint32_t* tables,
                                         size_t max_blocks, const int32_t* lengths,
                                         const float* tail_key, const float* tail_value,
                                         float* output, int page_dtype, float key_scale,
                                         float value_scale, helix_stream stream);
/* kernels::rope / cpu::rope_out (src/kernels/cpu/reference.cpp:490-533):
 * rotates the adjacent pairs (2i, 2i+1) of every head vector, out[2i] =
 * x[2i]*cos - x[2i+1]*sin, out[2i+1] = x[2i]*sin + x[2i+1]*cos, each product
 * and sum rounded to fp32 separately (bit-identical to the reference's CPU
 * path).  input, output [tokens, vectors, head_dim] (output == input allowed,
 * 8-byte aligned); cosine, sine [cache_rows, head_dim / 2].  positions NULL:
 * token t uses table row t (cache_rows must equal tokens, as the reference
 * requires); else row positions[t] (int32, device), and a position outside
 * [0, cache_rows) yields a NaN vector. */
int helix_rope(const float* input, float* output, size_t tokens, size_t vectors,
               size_t head_dim, const float* cosine, const float* sine, size_t cache_rows,
               const int32_t* positions, helix_stream stream);
/* Writes rows [count, kv_heads, head_dim] of keys/values into one layer's
 * pools at slots[i] = block * block_tokens + offset (negative: skipped). */
int helix_paged_append_slots(const float* keys, const float* values, float* key_blocks,
                             float* value_blocks, size_t physical_blocks, size_t kv_heads,
                             size_t block_tokens, size_t head_dim, const int64_t* slots,
                             size_t count, helix_stream stream);

/* -------------------------------------- chunked prefill (extension) ---- */
/* The reference's paged attention with a T-token tail (cuda_paged.cu:483-548,
 * paged_reference.cpp:173-384) for `batch` sequences at once, computed on
 * the matrix cores (fp32 MFMA): query row t of sequence b sees the
 * lengths[b] history tokens of row b of `tables` and chunk rows 0..t.
 *   query, output [batch, q_heads, tokens, head_dim];
 *   key_blocks, value_blocks [physical_blocks, kv_heads, block_tokens, head_dim];
 *   chunk_key, chunk_value [batch, kv_heads, tokens, head_dim];
 *   tables [batch, max_blocks] uint32; lengths [batch] int32.
 * Built for head_dim 128, 16-token pages and q_heads / kv_heads in
 * {1, 2, 4, 8}; any other geometry returns HELIX_UNSUPPORTED before a
 * launch. */
int helix_paged_prefill_attention(const float* query, size_t batch, size_t q_heads,
                                  size_t kv_heads, size_t tokens, size_t head_dim,
                                  const float* key_blocks, const float* value_blocks,
                                  size_t physical_blocks, size_t block_tokens,
                                  const uint32_t* tables, size_t max_blocks,
                                  const int32_t* lengths, const float* chunk_key,
                                  const float* chunk_value, float* output, helix_stream stream);
/* helix_paged_prefill_attention over bf16 or fp8 E4M3 pools (extension, as
 * helix_paged_decode_attention_typed): history keys and values are widened
 * from the pages, and the fp32 chunk rows rounded onto the pool's grid (the
 * values their pages hold once appended), so the result is the fp32
 * attention of the values the pages hold.  Runs the exact kernel (fp32
 * matrix cores).  HELIX_PAGE_F32 is exactly helix_paged_prefill_attention. */
int helix_paged_prefill_attention_typed(const float* query, size_t batch, size_t q_heads,
                                        size_t kv_heads, size_t tokens, size_t head_dim,
                                        const void* key_blocks, const void* value_blocks,
                                        size_t physical_blocks, size_t block_tokens,
                                        const uint32_t* tables, size_t max_blocks,
                                        const int32_t* lengths, const float* chunk_key,
                                        const float* chunk_value, float* output, int page_dtype,
                                        float key_scale, float value_scale, helix_stream stream);
/* Chunk append (PagedKvCache::append_layer_major, paged.cpp:721-871, for one
 * layer of `batch` sequences): rows [batch, kv_heads, tokens, head_dim] go
 * to slots[b * tokens + t] = block * block_tokens + offset (negative:
 * skipped). */
int helix_paged_append_chunk(const float* keys, const float* values, float* key_blocks,
                             float* value_blocks, size_t physical_blocks, size_t kv_heads,
                             size_t block_tokens, size_t head_dim, const int64_t* slots,
                             size_t batch, size_t tokens, helix_stream stream);

/* A decode driver over a cache: persistent device block tables for a fixed
 * set of sequences.  prepare() reserves one slot per sequence (allocating
 * pages), append_layer() writes it, attention_layer() attends over the
 * history before the step plus the tail.  prepare_chunk() reserves `tokens`
 * slots per sequence instead; append_layer() then takes [batch, kv_heads,
 * tokens, head_dim] rows and prefill_layer() runs the chunk attention.
 * Streams: any call may use any stream (it waits for the step's upload, and
 * the next prepare() waits for the last call's stream), but the calls of one
 * step share the batch's workspace and step buffers, so two attention or
 * prefill calls that overlap in time on different streams race; order them
 * (one stream, or events between streams), as a layer loop does. */
int helix_decode_batch_create(helix_paged_cache* cache, const helix_sequence* sequences,
                              size_t batch, size_t q_heads, size_t max_tokens,
                              size_t pages_per_split, helix_decode_batch** out);
int helix_decode_batch_prepare(helix_decode_batch* b, helix_stream stream);
/* append_layer() + attention_layer() of a one-token step in one decode launch
 * (keys/values [batch, kv_heads, 128] are both the rows to append and the
 * attention tail): the decode kernel writes each new token into its reserved
 * slot as it reads it, so the step needs no separate append launch. */
int helix_decode_batch_append_attention_layer(helix_decode_batch* b, size_t layer,
                                              const float* query, const float* keys,
                                              const float* values, float* output,
                                              helix_stream stream);
int helix_decode_batch_prepare_chunk(helix_decode_batch* b, size_t tokens, helix_stream stream);
int helix_decode_batch_append_layer(helix_decode_batch* b, size_t layer, const float* keys,
                                    const float* values, helix_stream stream);
/* append_layer() for every layer of the cache in one launch: keys/values
 * [layers, batch, kv_heads, tokens, head_dim].  The batched form of
 * CudaPagedKvCache::append (include/helix/kv_cache/cuda_paged.hpp:47-120,
 * src/kv_cache/cuda_paged.cpp:491-611), which commits one token's
 * [layers, kv_heads, head_dim] K/V after the forward pass has attended to it
 * as the uncommitted tail; the reference issues 2 * layers * kv_heads
 * device copies per sequence for it. */
int helix_decode_batch_append_all_layers(helix_decode_batch* b, const float* keys,
                                         const float* values, helix_stream stream);
/* Rotary embedding of a one-token step's query [batch, q_heads, head_dim]
 * and key [batch, kv_heads, head_dim] rows, in place and in one launch, each
 * sequence at its own position (its length before the step).  Replaces the
 * model's two kernels::rope launches per layer (src/model/cuda_llama.cpp:
 * 353-354); same arithmetic as helix_rope.  cosine/sine [cache_rows,
 * head_dim / 2] as detail::make_rope_cache builds them
 * (src/model/llama_common.cpp:22-47) for positions 0..cache_rows-1. */
int helix_decode_batch_rope(helix_decode_batch* b, float* query, float* key,
                            const float* cosine, const float* sine, size_t cache_rows,
                            helix_stream stream);
int helix_decode_batch_attention_layer(helix_decode_batch* b, size_t layer, const float* query,
                                       const float* tail_key, const float* tail_value,
                                       float* output, helix_stream stream);
/* The chunk attention of a prepare_chunk() step.  fp32 pages: the fp32
 * matrix cores, one 16-row tile per wavefront.  bf16 and fp8 pages: the bf16
 * matrix cores, page values exact in bf16 and the fp32 operand of each
 * product split into three exact bf16 terms (every product exact, fp32
 * accumulation).  Either way a work item that meets a special value (a NaN
 * in a row's accumulators or sum) is recomputed by the exact kernel in a
 * second launch, so the results follow the reference's special-value rules
 * within the fp32 tolerance.  The flags live in the batch's step buffer. */
int helix_decode_batch_prefill_layer(helix_decode_batch* b, size_t layer, const float* query,
                                     const float* chunk_key, const float* chunk_value,
                                     float* output, helix_stream stream);
int helix_decode_batch_tables(const helix_decode_batch* b, const uint32_t** tables,
                              const int32_t** lengths, const int64_t** slots,
                              size_t* max_blocks, size_t* pages_per_split);
/* Leading pages that every sequence of the prepared decode step shares and
 * that attention_layer() attends once for the whole batch on the matrix
 * cores (cascade; 0 when the step does not use it). */
int helix_decode_batch_shared_pages(const helix_decode_batch* b, size_t* out);
/* Measurement hook (no reference counterpart): when event (a hipEvent_t) is
 * non-NULL, every attention_layer() records it on its stream between the
 * main decode kernel and the merge kernel, so the dominant kernel can be
 * timed alone.  NULL turns it off. */
int helix_decode_batch_set_timing_event(helix_decode_batch* b, void* event);
void helix_decode_batch_destroy(helix_decode_batch* b);

/* ------------------------------------------------------ prefix cache ---- */
/* PagedPrefixCache (include/helix/kv_cache/prefix.hpp:66-112,
 * src/kv_cache/prefix.cpp): a bounded index from (namespace, exact token
 * IDs of a block-aligned prefix) to an anchor sequence the index owns in
 * the pool.  Namespace 0 is invalid.  Public calls take the index lock, then
 * the pool's (prefix.hpp:62-63). */
typedef struct helix_prefix_cache helix_prefix_cache;

/* PagedPrefixCacheConfig (prefix.hpp:34-37). */
typedef struct helix_prefix_config {
  size_t maximum_entries;
  size_t maximum_block_references;
} helix_prefix_config;

/* PrefixInsertStatus (prefix.hpp:39-43). */
typedef enum helix_prefix_insert_status {
  HELIX_PREFIX_INSERTED = 0,
  HELIX_PREFIX_ALREADY_PRESENT = 1,
  HELIX_PREFIX_REJECTED_TOO_LARGE = 2
} helix_prefix_insert_status;

/* PagedPrefixCacheStats (prefix.hpp:47-63), 64-bit. */
typedef struct helix_prefix_stats {
  uint64_t maximum_entries, maximum_block_references, entry_count, retained_tokens;
  uint64_t retained_block_references, peak_entries, peak_block_references;
  uint64_t lookup_count, hit_count, miss_count, insertion_count, duplicate_insertion_count;
  uint64_t rejected_insertion_count, eviction_count, erase_count;
} helix_prefix_stats;

/* PagedPrefixCache::PagedPrefixCache (prefix.cpp:124-139, 270-275) over the
 * device cache's pool; the index keeps the pool alive until destroyed. */
int helix_prefix_cache_create(helix_paged_cache* cache, const helix_prefix_config* config,
                              helix_prefix_cache** out);
/* The same index over host page bookkeeping only (no device memory); the
 * manager must outlive the index. */
int helix_prefix_cache_create_host(helix_block_manager* manager, const helix_prefix_config* config,
                                   helix_prefix_cache** out);
/* ~PagedPrefixCache (prefix.cpp:277-287): releases every retained anchor. */
void helix_prefix_cache_destroy(helix_prefix_cache* prefixes);
/* PagedPrefixCache::insert (prefix.cpp:296-358); *status is a
 * helix_prefix_insert_status. */
int helix_prefix_cache_insert(helix_prefix_cache* prefixes, uint64_t namespace_id,
                              const uint32_t* tokens, size_t count, helix_sequence source,
                              int* status);
/* PagedPrefixCache::lookup_longest (prefix.cpp:360-403): *hit = 1 and a new
 * sequence the caller must release, or *hit = 0. */
int helix_prefix_cache_lookup_longest(helix_prefix_cache* prefixes, uint64_t namespace_id,
                                      const uint32_t* tokens, size_t count,
                                      size_t maximum_prefix_tokens, int* hit,
                                      helix_sequence* sequence, size_t* matched_tokens);
/* contains / erase / evict_lru / clear (prefix.cpp:405-446). */
int helix_prefix_cache_contains(helix_prefix_cache* prefixes, uint64_t namespace_id,
                                const uint32_t* tokens, size_t count, int* out);
int helix_prefix_cache_erase(helix_prefix_cache* prefixes, uint64_t namespace_id,
                             const uint32_t* tokens, size_t count, int* erased);
int helix_prefix_cache_evict_lru(helix_prefix_cache* prefixes, int* evicted);
int helix_prefix_cache_clear(helix_prefix_cache* prefixes);
/* stats / config / block_tokens (prefix.cpp:448-463). */
int helix_prefix_cache_stats(helix_prefix_cache* prefixes, helix_prefix_stats* out);
int helix_prefix_cache_config(helix_prefix_cache* prefixes, helix_prefix_config* out);
int helix_prefix_cache_block_tokens(helix_prefix_cache* prefixes, size_t* out);

#ifdef __cplusplus
}
#endif

#endif /* HELIX_PAGED_H */
