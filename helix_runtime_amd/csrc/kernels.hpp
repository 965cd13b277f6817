// Device kernels of the paged-KV hot path (gfx950) and their host launchers.
//
// Every launcher takes plain device pointers and sizes, launches on the given
// stream and returns the hipError_t of the launch.  Shapes are validated by
// the callers (paged_cache.cpp / c_api.cpp) before anything is launched.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace helix::hip {

// XCDs of an MI355X.  The dispatcher hands consecutive workgroups of a launch
// to the XCDs in turn (workgroup i runs on XCD i % kXcds), and each XCD has
// its own L2: work items that read the same pages go to workgroups of one
// XCD so that the repeats hit that L2.
constexpr unsigned kXcds = 8;

// Pool geometry of one layer: [physical_blocks, kv_heads, block_tokens, dim].
struct PageGeometry {
  std::size_t physical_blocks;
  std::size_t kv_heads;
  std::size_t block_tokens;
  std::size_t head_dim;
};

// Element type of the pages: fp32 (the reference's format), bf16 (the
// appended fp32 value rounded to nearest even; NaN stays NaN) or fp8 E4M3
// with a key scale and a value scale (fp8.hpp).  Pool pointers are untyped
// where several may be passed; strides and offsets are in elements.  Rows
// appended and gather outputs are fp32 whatever the type.
enum class PageType : int { kF32 = 0, kBF16 = 1, kFP8 = 2 };
constexpr std::size_t page_element_bytes(PageType t) {
  return t == PageType::kBF16 ? 2 : t == PageType::kFP8 ? 1 : 4;
}
// The page type with its fp8 scales (1 and ignored for the other types).
struct PageFormat {
  PageType type = PageType::kF32;
  float k_scale = 1.0f;
  float v_scale = 1.0f;
  PageFormat() = default;
  PageFormat(PageType t, float k = 1.0f, float v = 1.0f)  // NOLINT: implicit from the type
      : type(t), k_scale(k), v_scale(v) {}
};

// One token for every layer.  src [layers, kv_heads, head_dim]; the token
// lands at (block, offset) of every layer pool.  Layer l's key pool starts at
// key_base + l * layer_stride (elements), values likewise.
hipError_t launch_append_token(const float* keys, const float* values, void* key_base,
                               void* value_base, std::size_t layer_stride, std::size_t layers,
                               const PageGeometry& g, std::uint32_t block, std::size_t offset,
                               hipStream_t stream, PageFormat type = PageFormat());

// Bulk layer-major append of `tokens` tokens.  layer_keys/layer_values are
// device arrays of `layers` device pointers, each [kv_heads, tokens, dim].
// blocks[i] is the physical block of logical block first_block + i.
// `vectorized` selects 128-bit accesses (every layer pointer 16-byte aligned
// and head_dim % 4 == 0, checked by the caller on the host copies).
hipError_t launch_append_bulk(const float* const* layer_keys, const float* const* layer_values,
                              void* key_base, void* value_base, std::size_t layer_stride,
                              std::size_t layers, const PageGeometry& g,
                              const std::uint32_t* blocks, std::size_t first_block,
                              std::size_t old_length, std::size_t tokens, hipStream_t stream,
                              bool vectorized, PageFormat type = PageFormat());

// Batched append: src [layers, count, kv_heads, tokens, dim];
// slots[i * tokens + t] is the flat slot block * block_tokens + offset of
// row (i, t) (negative rows skipped) in each of `layers` layer pools that
// start layer_stride page elements apart from key_pool / value_pool.
hipError_t launch_append_slots(const float* keys, const float* values, void* key_pool,
                               void* value_pool, const PageGeometry& g, const std::int64_t* slots,
                               std::size_t count, hipStream_t stream, std::size_t tokens = 1,
                               PageFormat type = PageFormat(), std::size_t layers = 1,
                               std::size_t layer_stride = 0);

// Rotary embedding (cpu::rope_out, bit-exact) of up to two tensors
// [rows, vectors, head_dim] whose rows share positions; row r uses cache row
// positions[r] (positions == nullptr: row r).  rows * vectors * head_dim / 2
// summed over both must stay below 2^32.
struct RopeTensor {
  const float* input = nullptr;
  float* output = nullptr;
  std::size_t vectors = 0;
};
hipError_t launch_rope(const RopeTensor& a, const RopeTensor& b, std::size_t rows,
                       std::size_t head_dim, const float* cosine, const float* sine,
                       std::size_t cache_rows, const std::int32_t* positions, hipStream_t stream);

// Gather one layer of one sequence into fp32 [kv_heads, dest_tokens, dim]:
// tokens [first_token, first_token + length) to rows [0, length).
hipError_t launch_gather(const void* key_pool, const void* value_pool, const PageGeometry& g,
                         const std::uint32_t* blocks, std::size_t length, float* keys_out,
                         float* values_out, std::size_t dest_tokens, hipStream_t stream,
                         PageFormat type = PageFormat(), std::size_t first_token = 0);

// Copy the first `tokens` token rows of block `from` into block `to` for
// every layer and head (copy-on-write of a partial shared page).
hipError_t launch_page_copy(void* key_base, void* value_base, std::size_t layer_stride,
                            std::size_t layers, const PageGeometry& g, std::uint32_t from,
                            std::uint32_t to, std::size_t tokens, hipStream_t stream,
                            PageFormat type = PageFormat());

// Scatter (row, column, value) triples into a [rows, cols] uint32 table.
hipError_t launch_table_updates(std::uint32_t* tables, std::size_t cols,
                                const std::uint32_t* updates, std::size_t count,
                                hipStream_t stream);

// ------------------------------------------------------------- decode ----
// Batched one-token decode with an uncommitted tail: split-K over pages
// (explicit pages_per_split) or the persistent stream kernel (0), each
// followed by a merge of the partials.
//   query      [batch, q_heads, 128]
//   tables     [batch, max_blocks] physical block IDs
//   lengths    [batch] committed history tokens per sequence
//   tail_key / tail_value [batch, kv_heads, 128]
//   out        [batch, q_heads, 128]
//   workspace  decode_workspace_bytes(...) bytes of split partials
//   items      exact work-item count (decode_items) or 0 for the upper bound
struct DecodeArgs {
  const float* query;
  const float* key_pool;
  const float* value_pool;
  const std::uint32_t* tables;
  const std::int32_t* lengths;
  const float* tail_key;
  const float* tail_value;
  float* out;
  void* workspace;
  std::size_t batch;
  std::size_t q_heads;
  std::size_t kv_heads;
  std::size_t max_blocks;
  std::size_t physical_blocks;
  std::size_t pages_per_split;
  std::size_t items;
  // Optional: recorded on the stream between the main kernel and the merge
  // (measurement of the dominant kernel alone).
  hipEvent_t between_event = nullptr;
  // Cascade (stream mode only): the first shared_pages pages of every
  // sequence are the same physical pages (row 0 of tables); they are attended
  // once for all sequences on the matrix cores and the stream kernel covers
  // the rest.  0: off.
  std::size_t shared_pages = 0;
  // Element type of key_pool / value_pool (and the append pools): bf16 and
  // fp8 pages are read through the same pointers, typed nominally as float.
  // Stream mode only for those types.
  PageFormat page_type;
  // Optional second stream for the cascade prefix pass: when set (with the
  // two events), the prefix runs on side_stream concurrently with the
  // stream kernel, which then takes one wavefront per SIMD and leaves the
  // other half of each register file to the prefix workgroups.  The merge
  // waits for both; between_event then marks the end of the stream kernel
  // only.
  hipStream_t side_stream = nullptr;
  hipEvent_t fork_event = nullptr;
  hipEvent_t join_event = nullptr;
  // Fused append (stream mode only): also write tail row b to physical slot
  // append_slots[b] (block * 16 + offset, negative: skipped) of these pools.
  const std::int64_t* append_slots = nullptr;
  float* append_key_pool = nullptr;
  float* append_value_pool = nullptr;
  // Stream mode without a cascade: partials laid out for the launch's own
  // wavefront count (compact_decode_workspace_bytes) instead of the
  // worst-case layout of decode_workspace_bytes.
  bool compact_layout = false;
};

constexpr std::size_t kDecodeHeadDim = 128;
constexpr std::size_t kDecodeBlockTokens = 16;
// pages_per_split == 0 selects the persistent stream kernel (the default):
// one wavefront per resident slot streams an equal share of all pages.
constexpr std::size_t kDefaultPagesPerSplit = 0;
// Largest split count per sequence the split-mode merge kernel's LDS holds.
constexpr std::size_t kMaxDecodeSplits = 4096;
// Most wavefronts a stream-mode launch uses (sizes its partial slots).
constexpr std::size_t kMaxStreamWaves = 4096;

std::size_t decode_max_splits(std::size_t max_blocks, std::size_t pages_per_split);
std::size_t decode_workspace_bytes(std::size_t batch, std::size_t q_heads, std::size_t kv_heads,
                                   std::size_t max_blocks, std::size_t pages_per_split);
// Work items of one launch for host-known lengths.
std::size_t decode_items(const std::int32_t* lengths, std::size_t batch, std::size_t kv_heads,
                         std::size_t max_blocks, std::size_t pages_per_split);
hipError_t launch_decode_workspace_init(void* workspace, std::size_t bytes, hipStream_t stream);
bool decode_group_supported(std::size_t group);
hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream);
// Workspace of a stream-mode decode with compact_layout (no cascade) over
// pages of `type`.
std::size_t compact_decode_workspace_bytes(std::size_t batch, std::size_t q_heads,
                                           std::size_t kv_heads,
                                           PageType type = PageType::kF32);

// ------------------------------------- reference-shaped one-sequence decode ----
// One query row per head (the reference's per-layer model call) over pages of
// head_dim 128 and 16 tokens, query groups 1/2/4/8, in one launch that also
// leaves the softmax probabilities in the score workspace [q_heads, keys]
// as the reference does: keys [0, visible) from the pages, then with `tail`
// the tail row as key `visible`; keys past those get probability 0.
struct RefDecodeArgs {
  const float* query;        // [q_heads, 128]
  const float* key_pool;     // [physical_blocks, kv_heads, 16, 128]
  const float* value_pool;
  const std::uint32_t* table;  // ceil(visible / 16) entries
  const float* tail_key;     // [kv_heads, 128] when tail
  const float* tail_value;
  float* out;                // [q_heads, 128]
  float* probs;              // [q_heads, keys]
  std::size_t q_heads, kv_heads, physical_blocks;
  std::size_t visible, keys;
  bool tail;
  // ref_decode_plan(...).scratch_bytes of device memory for the partials of
  // calls that take more than one workgroup per kv head (those then run a
  // second, merging launch).  Calls that share a scratch must run in order
  // (one stream).
  void* scratch;
  // Optional: recorded between the two launches (timing of the first).
  hipEvent_t between_event = nullptr;
};
struct RefDecodePlan {
  std::size_t chunks = 0;        // workgroups per kv head
  std::size_t ppw = 0;           // pages per wavefront
  std::size_t scratch_bytes = 0;
};
// Workspace keys one merging or normalising workgroup rewrites, and the
// longest workspace row the fast reference-shaped routes take (their
// grids' second dimension stays within 65535).
constexpr std::size_t kRefNormKeys = 2048;
constexpr std::size_t kRefDecodeMaxKeys = 65535 * kRefNormKeys;
RefDecodePlan ref_decode_plan(std::size_t q_heads, std::size_t kv_heads, std::size_t visible,
                              bool tail);
hipError_t launch_ref_decode(const RefDecodeArgs& a, const RefDecodePlan& plan,
                             hipStream_t stream);

// ------------------------------------------------------------ generic ----
// Reference-shaped paged attention for any geometry (one query row per
// workgroup).  Materialises probabilities into workspace [q_heads, queries,
// history + tail] exactly like the reference's score workspace contract.
struct GenericArgs {
  const float* query;        // [q_heads, queries, key_dim]
  const float* key_blocks;   // [physical, kv_heads, block_tokens, key_dim]
  const float* value_blocks; // [physical, kv_heads, block_tokens, value_dim]
  const std::uint32_t* table;
  const float* tail_key;     // [kv_heads, tail, key_dim] or null
  const float* tail_value;   // [kv_heads, tail, value_dim] or null
  float* out;                // [q_heads, queries, value_dim]
  float* workspace;          // [q_heads, queries, history + tail]
  std::size_t q_heads, kv_heads, queries, key_dim, value_dim;
  std::size_t block_tokens, physical_blocks;
  std::size_t history, tail, offset;
};

hipError_t launch_generic(const GenericArgs& a, hipStream_t stream);

// ------------------------------------------------------- chunked prefill ----
// Batched chunked-prefill attention (MFMA): every sequence b attends with
// `tokens` query rows to its paged history (lengths[b] tokens through row b
// of tables) plus its chunk, causally inside the chunk.  Shapes: query and
// out [batch, q_heads, tokens, 128]; chunk_key/value [batch, kv_heads,
// tokens, 128]; pools [physical_blocks, kv_heads, 16, 128].
struct PrefillArgs {
  const float* query;
  const float* key_pool;
  const float* value_pool;
  const std::uint32_t* tables;
  const std::int32_t* lengths;
  const float* chunk_key;
  const float* chunk_value;
  float* out;
  std::size_t batch, q_heads, kv_heads, tokens, max_blocks, physical_blocks;
  // Optional launch order of the batch * kv_heads * ceil(tokens / positions
  // per block) work items, packed (b * kv_heads + kvh) * blocks + block.
  const std::uint32_t* order = nullptr;
  // bf16 / fp8 pages: history keys/values are widened and the chunk rows
  // rounded onto the page grid (the values their pages hold once appended).
  PageFormat page_type;
  // bf16 / fp8 pages: one word per launched work item.  Given, the launch
  // runs on the bf16 matrix cores and redoes exactly the items that met a
  // special value (a NaN score, a non-finite value row that some row
  // masks); the words are written by the launch itself.
  std::uint32_t* redo = nullptr;
  // One sequence whose history is a host value: lengths == nullptr.
  std::int32_t single_length = 0;
  // fp32 pages, exact kernel, one sequence: also write the softmax
  // probabilities of every query row to probs [q_heads, tokens, prob_keys],
  // 0 for keys the row does not see -- the reference's score workspace
  // contract (a second launch turns the written scores into probabilities).
  float* probs = nullptr;
  std::size_t prob_keys = 0;
  // With probs (one sequence, lengths == nullptr): the key blocks of each
  // work item are split into prob_splits ranges (prefill_prob_splits), and
  // scratch of q_heads * tokens * prob_splits * 2 floats (prob_ml) and
  // * 128 floats (prob_o) holds each range's row maximum, sum and
  // unnormalised output.
  std::size_t prob_splits = 1;
  float* prob_ml = nullptr;
  float* prob_o = nullptr;
};

// Shared-prefix attention for a decode batch (cascade): every query row of
// every sequence against the first shared_pages pages of `table`, leaving a
// partial (m, l, o) per (sequence, kv head) unit at prefix_slot0 + kvh *
// batch + b of the decode workspace partials.
struct CascadePrefixArgs {
  const float* query;
  const float* key_pool;
  const float* value_pool;
  const std::uint32_t* table;
  float* part_o;
  float* part_ml;
  std::size_t batch, q_heads, kv_heads, shared_pages, physical_blocks, prefix_slot0;
  PageFormat page_type;
};
hipError_t launch_cascade_prefix(const CascadePrefixArgs& a, hipStream_t stream);
// The shared prefix is split into key chunks (each leaving its own partial
// per unit, at slot prefix_slot0 + chunk * units + unit).
constexpr std::size_t kMaxCascadeChunks = 16;
// Query groups up to this size run the cascade prefix pass and the stream
// kernel as one launch; larger groups put the prefix pass on a side stream
// (DecodeArgs::side_stream).
constexpr std::size_t kCascadeFusedMaxGroup = 4;
std::size_t cascade_chunk_pages(std::size_t shared_pages, std::size_t batch, std::size_t group,
                                std::size_t kv_heads);

bool prefill_group_supported(std::size_t group);
// Chunk positions one prefill work item covers for a query group size.
std::size_t prefill_position_block(std::size_t group);
hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream);
// Key ranges per work item of a one-sequence probability prefill (1..8).
std::size_t prefill_prob_splits(std::size_t q_heads, std::size_t kv_heads, std::size_t tokens,
                                std::size_t keys, int cus);
// CUs of the current device, looked up once per device.
int device_cus();

}  // namespace helix::hip
