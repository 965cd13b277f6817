#include "paged_cache.hpp"

#include "kernels.hpp"
#include "status.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <string>
#include <utility>

namespace helix {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fail(Status::kRuntime, std::string(what) + ": " + hipGetErrorString(e));
  }
}

DeviceBuffer::DeviceBuffer(std::size_t bytes, int device) : bytes_(bytes) {
  if (bytes == 0) return;
  DeviceGuard guard(device);
  const hipError_t e = hipMalloc(&ptr_, bytes);
  if (e != hipSuccess) {
    ptr_ = nullptr;
    (void)hipGetLastError();
    fail(e == hipErrorOutOfMemory ? Status::kResourceExhausted : Status::kRuntime,
         std::string("device allocation of ") + std::to_string(bytes) +
             " bytes failed: " + hipGetErrorString(e));
  }
}

DeviceBuffer::~DeviceBuffer() {
  if (ptr_ != nullptr) (void)hipFree(ptr_);
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept
    : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
  if (this != &o) {
    if (ptr_ != nullptr) (void)hipFree(ptr_);
    ptr_ = std::exchange(o.ptr_, nullptr);
    bytes_ = std::exchange(o.bytes_, 0);
  }
  return *this;
}

PinnedBuffer::PinnedBuffer(std::size_t bytes) {
  hip_check(hipHostMalloc(&ptr_, bytes, hipHostMallocDefault), "hipHostMalloc");
}

PinnedBuffer::~PinnedBuffer() {
  if (ptr_ != nullptr) (void)hipHostFree(ptr_);
}

PinnedBuffer::PinnedBuffer(PinnedBuffer&& o) noexcept : ptr_(std::exchange(o.ptr_, nullptr)) {}

PinnedBuffer& PinnedBuffer::operator=(PinnedBuffer&& o) noexcept {
  if (this != &o) {
    if (ptr_ != nullptr) (void)hipHostFree(ptr_);
    ptr_ = std::exchange(o.ptr_, nullptr);
  }
  return *this;
}

DeviceGuard::DeviceGuard(int device) {
  hip_check(hipGetDevice(&previous_), "hipGetDevice");
  if (previous_ != device) hip_check(hipSetDevice(device), "hipSetDevice");
}

DeviceGuard::~DeviceGuard() {
  int current = -1;
  if (hipGetDevice(&current) == hipSuccess && current != previous_) (void)hipSetDevice(previous_);
}

namespace {

std::size_t pool_elements(const PagedConfig& c) {
  return c.physical_blocks * c.kv_heads * c.block_tokens * c.head_dimension;
}

hip::PageGeometry geometry(const PagedConfig& c) {
  return hip::PageGeometry{c.physical_blocks, c.kv_heads, c.block_tokens, c.head_dimension};
}

void check_device(int device) {
  check(device >= 0, Status::kInvalidArgument, "device index must be non-negative");
  int count = 0;
  hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
  check(device < count, Status::kInvalidArgument, "device index exceeds the visible devices");
}

bool ranges_overlap(const void* a, std::size_t an, const void* b, std::size_t bn) {
  if (an == 0 || bn == 0 || a == nullptr || b == nullptr) return false;
  const auto x = reinterpret_cast<std::uintptr_t>(a);
  const auto y = reinterpret_cast<std::uintptr_t>(b);
  return x < y + bn && y < x + an;
}

// Synchronises the stream after enqueued work; a failure leaves the device
// state uncertain and poisons the cache (src/kv_cache/cuda_paged.cpp:577-583).
void synchronize_or_poison(CacheState& s, hipStream_t stream, const char* what) {
  const hipError_t e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    s.poisoned = true;
    fail(Status::kRuntime, std::string(what) + ": stream synchronisation failed: " +
                               hipGetErrorString(e));
  }
}

}  // namespace

CacheState::CacheState(const PagedConfig& config, int dev, hip::PageFormat type)
    : manager(config, hip::page_element_bytes(type.type)), device((check_device(dev), dev)),
      page_type(type) {
  layer_elements = pool_elements(config);
  const std::size_t bytes = manager.stats().bytes_reserved;
  slab = DeviceBuffer(bytes, device);
}

bool CacheState::overlaps_pool(const void* p, std::size_t bytes) const {
  return ranges_overlap(p, bytes, slab.data(), slab.size());
}

void CacheState::require_healthy(const char* op) const {
  check(!poisoned, Status::kRuntime,
        std::string(op) + ": cache is unusable after a device stream could not be drained");
}

void CacheState::require_sequence(std::uint64_t id, std::uint64_t cache_id, const char* op) const {
  check(id != 0 && cache_id == manager.cache_id(), Status::kInvalidArgument,
        std::string(op) + ": sequence handle belongs to another cache or is empty");
  check(manager.contains(id), Status::kInvalidArgument,
        std::string(op) + ": sequence is unknown or was already released");
}

void* CacheState::staging_bytes(std::size_t bytes) {
  if (staging.size() < bytes) {
    staging = DeviceBuffer(std::max<std::size_t>(bytes, 4096), device);
  }
  return staging.data();
}

DevicePagedCache::DevicePagedCache(const PagedConfig& config, int device, hip::PageFormat page_type)
    : state_(std::make_shared<CacheState>(config, device, page_type)) {}

std::uint64_t DevicePagedCache::create_sequence() {
  std::scoped_lock lock(state_->mutex);
  state_->require_healthy("create_sequence");
  return state_->manager.create_sequence();
}

std::uint64_t DevicePagedCache::fork_sequence(std::uint64_t sequence, std::uint64_t cache_id,
                                              std::size_t prefix, bool allow_copy_on_write,
                                              hipStream_t stream) {
  CacheState& s = *state_;
  std::scoped_lock lock(s.mutex);
  s.require_healthy("fork_sequence");
  s.require_sequence(sequence, cache_id, "fork_sequence");
  const ForkPlan plan = s.manager.plan_fork(sequence, prefix, allow_copy_on_write);
  if (plan.copy_on_write) {
    DeviceGuard guard(s.device);
    const PagedConfig& c = s.manager.config();
    hip_check(hip::launch_page_copy(s.key_pool(0), s.value_pool(0), s.layer_stride(), c.layers,
                                    geometry(c), plan.cow_from, plan.cow_to, plan.cow_tokens,
                                    stream, s.page_type),
              "fork_sequence copy-on-write launch");
    synchronize_or_poison(s, stream, "fork_sequence");
  }
  return s.manager.commit_fork(plan);
}

void DevicePagedCache::append(std::uint64_t sequence, std::uint64_t cache_id, const float* keys,
                              const float* values, hipStream_t stream) {
  CacheState& s = *state_;
  std::scoped_lock lock(s.mutex);
  s.require_healthy("append");
  s.require_sequence(sequence, cache_id, "append");
  const PagedConfig& c = s.manager.config();
  check(keys != nullptr && values != nullptr, Status::kInvalidArgument,
        "append: token keys and values must be non-null device pointers");
  const std::size_t bytes = c.layers * c.kv_heads * c.head_dimension * sizeof(float);
  check(!s.overlaps_pool(keys, bytes) && !s.overlaps_pool(values, bytes),
        Status::kInvalidArgument, "append: input must not alias cache-owned page storage");
  const AppendPlan plan = s.manager.plan_append(sequence, 1);
  const std::uint64_t slot = plan.slot(0, c.block_tokens);
  DeviceGuard guard(s.device);
  hip_check(hip::launch_append_token(keys, values, s.key_pool(0), s.value_pool(0),
                                     s.layer_stride(), c.layers, geometry(c),
                                     static_cast<std::uint32_t>(slot / c.block_tokens),
                                     slot % c.block_tokens, stream, s.page_type),
            "append launch");
  synchronize_or_poison(s, stream, "append");
  s.manager.commit_append(plan);
}

void DevicePagedCache::append_layer_major(std::uint64_t sequence, std::uint64_t cache_id,
                                          const float* const* layer_keys,
                                          const float* const* layer_values, std::size_t tokens,
                                          hipStream_t stream) {
  CacheState& s = *state_;
  std::scoped_lock lock(s.mutex);
  s.require_healthy("append_layer_major");
  s.require_sequence(sequence, cache_id, "append_layer_major");
  const PagedConfig& c = s.manager.config();
  check(layer_keys != nullptr && layer_values != nullptr, Status::kInvalidArgument,
        "append_layer_major requires one key/value tensor per layer");
  check(tokens != 0, Status::kInvalidArgument, "append_layer_major token count must be positive");
  const std::size_t bytes = c.kv_heads * tokens * c.head_dimension * sizeof(float);
  bool aligned = c.head_dimension % 4 == 0;
  for (std::size_t l = 0; l < c.layers; ++l) {
    check(layer_keys[l] != nullptr && layer_values[l] != nullptr, Status::kInvalidArgument,
          "append_layer_major layer tensors must be non-null device pointers");
    check(!s.overlaps_pool(layer_keys[l], bytes) && !s.overlaps_pool(layer_values[l], bytes),
          Status::kInvalidArgument, "append_layer_major input must not alias cache-owned pages");
    aligned = aligned && (reinterpret_cast<std::uintptr_t>(layer_keys[l]) & 15u) == 0 &&
              (reinterpret_cast<std::uintptr_t>(layer_values[l]) & 15u) == 0;
  }
  const AppendPlan plan = s.manager.plan_append(sequence, tokens);

  // Upload [layer key ptrs | layer value ptrs | physical blocks] once.
  std::vector<unsigned char> host(2 * c.layers * sizeof(void*) +
                                  plan.blocks.size() * sizeof(std::uint32_t));
  std::memcpy(host.data(), layer_keys, c.layers * sizeof(void*));
  std::memcpy(host.data() + c.layers * sizeof(void*), layer_values, c.layers * sizeof(void*));
  std::memcpy(host.data() + 2 * c.layers * sizeof(void*), plan.blocks.data(),
              plan.blocks.size() * sizeof(std::uint32_t));
  DeviceGuard guard(s.device);
  auto* dev = static_cast<unsigned char*>(s.staging_bytes(host.size()));
  hip_check(hipMemcpyAsync(dev, host.data(), host.size(), hipMemcpyHostToDevice, stream),
            "append_layer_major upload");
  const auto* dkeys = reinterpret_cast<const float* const*>(dev);
  const auto* dvalues = reinterpret_cast<const float* const*>(dev + c.layers * sizeof(void*));
  const auto* dblocks = reinterpret_cast<const std::uint32_t*>(dev + 2 * c.layers * sizeof(void*));
  hip_check(hip::launch_append_bulk(dkeys, dvalues, s.key_pool(0), s.value_pool(0),
                                    s.layer_stride(), c.layers, geometry(c), dblocks,
                                    plan.first_block, plan.old_length, tokens, stream, aligned,
                                    s.page_type),
            "append_layer_major launch");
  synchronize_or_poison(s, stream, "append_layer_major");
  s.manager.commit_append(plan);
}

void DevicePagedCache::release(std::uint64_t sequence, std::uint64_t cache_id) {
  std::scoped_lock lock(state_->mutex);
  state_->require_sequence(sequence, cache_id, "release_sequence");
  state_->manager.release(sequence);
  state_->releases.fetch_add(1, std::memory_order_release);
}

void DevicePagedCache::copy_layer_out(std::uint64_t sequence, std::uint64_t cache_id,
                                      std::size_t layer, std::size_t expected_length,
                                      float* keys_out, float* values_out, std::size_t dest_tokens,
                                      hipStream_t stream) {
  CacheState& s = *state_;
  std::scoped_lock lock(s.mutex);
  s.require_healthy("copy_layer_out");
  s.require_sequence(sequence, cache_id, "copy_layer_out");
  const PagedConfig& c = s.manager.config();
  const std::size_t length = s.manager.length(sequence);
  check(expected_length == std::numeric_limits<std::size_t>::max() || expected_length == length,
        Status::kInvalidArgument,
        "copy_layer_prefix_out cached length does not match the caller's expected length");
  check(layer < c.layers, Status::kOutOfRange, "copy_layer_out layer index is out of range");
  check(dest_tokens >= length, Status::kInvalidArgument,
        "copy_layer_out output token capacity is smaller than the cached history");
  const std::size_t bytes = c.kv_heads * dest_tokens * c.head_dimension * sizeof(float);
  check(length == 0 || (keys_out != nullptr && values_out != nullptr), Status::kInvalidArgument,
        "copy_layer_out outputs must be non-null device pointers");
  check(!ranges_overlap(keys_out, bytes, values_out, bytes), Status::kInvalidArgument,
        "copy_layer_out key and value outputs must not alias");
  check(!s.overlaps_pool(keys_out, bytes) && !s.overlaps_pool(values_out, bytes),
        Status::kInvalidArgument, "copy_layer_out outputs must not alias cache-owned pages");
  if (length == 0) return;
  const std::vector<std::uint32_t>& blocks = s.manager.blocks(sequence);
  DeviceGuard guard(s.device);
  auto* dev = static_cast<std::uint32_t*>(s.staging_bytes(blocks.size() * sizeof(std::uint32_t)));
  hip_check(hipMemcpyAsync(dev, blocks.data(), blocks.size() * sizeof(std::uint32_t),
                           hipMemcpyHostToDevice, stream),
            "copy_layer_out table upload");
  hip_check(hip::launch_gather(s.key_pool(layer), s.value_pool(layer), geometry(c), dev, length,
                               keys_out, values_out, dest_tokens, stream, s.page_type),
            "copy_layer_out launch");
  synchronize_or_poison(s, stream, "copy_layer_out");
}

// ----------------------------------------------------------- DecodeView ----
DecodeView::DecodeView(std::shared_ptr<CacheState> state, std::uint64_t sequence,
                       std::uint64_t cache_id)
    : state_(std::move(state)), lock_(state_->mutex) {
  state_->require_healthy("read_sequence");
  state_->require_sequence(sequence, cache_id, "read_sequence");
  length_ = state_->manager.length(sequence);
  blocks_ = state_->manager.blocks(sequence);
  if (!blocks_.empty()) {
    // Synchronous upload, as PagedBlockTable does (src/kv_cache/
    // cuda_block_table.cpp:44-46).
    table_ = DeviceBuffer(blocks_.size() * sizeof(std::uint32_t), state_->device);
    DeviceGuard guard(state_->device);
    hip_check(hipMemcpy(table_.data(), blocks_.data(), table_.size(), hipMemcpyHostToDevice),
              "read_sequence table upload");
  }
  valid_ = true;
}

void DecodeView::require_valid(const char* op) const {
  check(valid_, Status::kInvalidArgument, std::string(op) + ": decode view is poisoned");
}

std::size_t DecodeView::length() const {
  require_valid("DecodeView::length");
  return length_;
}

const std::vector<std::uint32_t>& DecodeView::physical_blocks() const {
  require_valid("DecodeView::physical_blocks");
  return blocks_;
}

const std::uint32_t* DecodeView::device_table() const {
  require_valid("DecodeView::block_table");
  return static_cast<const std::uint32_t*>(table_.data());
}

float* DecodeView::key_pool(std::size_t layer) const {
  require_valid("DecodeView::layer_key_blocks");
  check(layer < state_->manager.config().layers, Status::kOutOfRange, "layer is out of range");
  return state_->key_pool(layer);
}

float* DecodeView::value_pool(std::size_t layer) const {
  require_valid("DecodeView::layer_value_blocks");
  check(layer < state_->manager.config().layers, Status::kOutOfRange, "layer is out of range");
  return state_->value_pool(layer);
}

// CudaPagedKvCache::DecodeView::poison_after_consumer_failure
// (src/kv_cache/cuda_paged.cpp:441-452): the cache stops admitting work and
// the device table is kept alive until the cache itself is destroyed.
void DecodeView::poison() noexcept {
  if (!valid_) return;
  state_->poisoned = true;
  valid_ = false;
  static_cast<void>(table_.data());
  state_->staging = std::move(table_);  // quarantined with the cache
}

// ---------------------------------------------------------- DecodeBatch ----
namespace {
constexpr std::size_t align8(std::size_t n) { return (n + 7) & ~std::size_t{7}; }
}  // namespace

DecodeBatch::DecodeBatch(std::shared_ptr<CacheState> state, const std::uint64_t* sequences,
                         const std::uint64_t* cache_ids, std::size_t batch, std::size_t q_heads,
                         std::size_t max_tokens, std::size_t pages_per_split)
    : state_(std::move(state)), q_heads_(q_heads) {
  CacheState& s = *state_;
  std::scoped_lock lock(s.mutex);
  s.require_healthy("decode batch");
  const PagedConfig& c = s.manager.config();
  check(batch != 0, Status::kInvalidArgument, "decode batch must hold at least one sequence");
  check(c.head_dimension == hip::kDecodeHeadDim && c.block_tokens == hip::kDecodeBlockTokens,
        Status::kUnsupported, "batched decode requires head_dim 128 and 16-token pages");
  check(q_heads != 0 && q_heads % c.kv_heads == 0 &&
            hip::decode_group_supported(q_heads / c.kv_heads),
        Status::kUnsupported, "batched decode supports query groups of 1, 2, 4 or 8 heads");
  max_blocks_ = (max_tokens + c.block_tokens - 1) / c.block_tokens;
  check(max_blocks_ != 0, Status::kInvalidArgument, "decode batch max_tokens must be positive");
  sequences_.assign(sequences, sequences + batch);
  std::size_t total_pages = 0;
  for (std::size_t i = 0; i < batch; ++i) {
    s.require_sequence(sequences[i], cache_ids[i], "decode batch");
    for (std::size_t k = 0; k < i; ++k) {
      check(sequences[k] != sequences[i], Status::kInvalidArgument,
            "decode batch lists a sequence twice");
    }
    check(s.manager.length(sequences[i]) < max_tokens, Status::kInvalidArgument,
          "decode batch max_tokens leaves no room for the next token");
    total_pages += s.manager.blocks(sequences[i]).size();
  }
  static_cast<void>(total_pages);
  pages_per_split_ = pages_per_split != 0 ? pages_per_split : hip::kDefaultPagesPerSplit;
  check(!s.reduced() || pages_per_split_ == 0, Status::kUnsupported,
        "decode batch: bf16 and fp8 pages decode in stream mode only (pages_per_split 0)");
  check(hip::decode_max_splits(max_blocks_, pages_per_split_) <= hip::kMaxDecodeSplits,
        Status::kUnsupported, "decode batch: max_tokens / pages_per_split above 4096 splits");
  host_lengths_.assign(batch, 0);

  DeviceGuard guard(s.device);
  std::vector<std::uint32_t> host(batch * max_blocks_, 0);
  for (std::size_t i = 0; i < batch; ++i) {
    const auto& blocks = s.manager.blocks(sequences[i]);
    std::copy(blocks.begin(), blocks.end(), host.begin() + static_cast<std::ptrdiff_t>(i * max_blocks_));
  }
  tables_ = DeviceBuffer(host.size() * sizeof(std::uint32_t), s.device);
  hip_check(hipMemcpy(tables_.data(), host.data(), tables_.size(), hipMemcpyHostToDevice),
            "decode batch table upload");
  mirrored_.resize(batch);
  for (std::size_t i = 0; i < batch; ++i) mirrored_[i] = s.manager.blocks(sequences[i]).size();
  mirror_ = std::move(host);
  workspace_ = DeviceBuffer(
      hip::decode_workspace_bytes(batch, q_heads, c.kv_heads, max_blocks_, pages_per_split_),
      s.device);
  hip_check(hip::launch_decode_workspace_init(workspace_.data(), workspace_.size(), nullptr),
            "decode batch workspace init");
  hip_check(hipDeviceSynchronize(), "decode batch workspace init");
  for (int i = 0; i < 2; ++i) {
    hip_check(hipEventCreateWithFlags(&uploaded_[i], hipEventDisableTiming), "hipEventCreate");
  }
  hip_check(hipEventCreateWithFlags(&order_event_, hipEventDisableTiming), "hipEventCreate");
  reserve_step(1);
}

DecodeBatch::~DecodeBatch() {
  // Destructors must not throw: switch devices without the checked guard.
  int previous = -1;
  const bool switched = hipGetDevice(&previous) == hipSuccess && previous != state_->device &&
                        hipSetDevice(state_->device) == hipSuccess;
  for (hipEvent_t e : uploaded_) {
    if (e != nullptr) {
      (void)hipEventSynchronize(e);
      (void)hipEventDestroy(e);
    }
  }
  if (side_stream_ != nullptr) {
    (void)hipStreamSynchronize(side_stream_);
    (void)hipStreamDestroy(side_stream_);
  }
  for (hipEvent_t e : {fork_event_, join_event_, order_event_}) {
    if (e != nullptr) (void)hipEventDestroy(e);
  }
  if (switched) (void)hipSetDevice(previous);
}

const std::uint32_t* DecodeBatch::tables() const {
  return static_cast<const std::uint32_t*>(tables_.data());
}
const std::int32_t* DecodeBatch::lengths() const {
  return static_cast<const std::int32_t*>(step_.data());
}
const std::int64_t* DecodeBatch::slots() const {
  return reinterpret_cast<const std::int64_t*>(static_cast<const unsigned char*>(step_.data()) +
                                               align8(batch() * sizeof(std::int32_t)));
}

// Step buffers for `tokens` slots per sequence: lengths [B] int32, slots
// [B, tokens] int64, up to B * max_blocks table updates of 3 words (a step
// uploads the entries a member gained since the previous step, inside or
// outside the batch), and for chunks the prefill work-item order, in one
// device buffer and two pinned staging copies; after them, device only, one
// redo word per prefill work item (written by the bf16 / fp8 prefill).
std::size_t DecodeBatch::order_offset(std::size_t tokens) const {
  const std::size_t B = batch();
  const std::size_t max_updates = B * max_blocks_;
  return align8(B * sizeof(std::int32_t)) + B * tokens * sizeof(std::int64_t) +
         3 * max_updates * sizeof(std::uint32_t);
}

std::size_t DecodeBatch::prefill_items(std::size_t tokens) const {
  const std::size_t pw = hip::prefill_position_block(q_heads_ / state_->manager.config().kv_heads);
  return batch() * state_->manager.config().kv_heads * ((tokens + pw - 1) / pw);
}

void DecodeBatch::reserve_step(std::size_t tokens) {
  if (tokens <= step_capacity_) return;
  const std::size_t bytes =
      order_offset(tokens) + 2 * prefill_items(tokens) * sizeof(std::uint32_t);
  for (hipEvent_t e : uploaded_) hip_check(hipEventSynchronize(e), "decode batch staging wait");
  DeviceGuard guard(state_->device);
  // The device buffer may still be read by queued kernels of earlier steps.
  hip_check(hipDeviceSynchronize(), "decode batch step resize");
  step_ = DeviceBuffer(bytes, state_->device);
  for (auto& pinned : pinned_) pinned = PinnedBuffer(bytes);
  step_bytes_ = bytes;
  step_capacity_ = tokens;
}

void DecodeBatch::prepare(hipStream_t stream, std::size_t tokens) {
  CacheState& s = *state_;
  std::scoped_lock lock(s.mutex);
  prepared_ = false;
  step_tokens_ = 0;
  s.require_healthy("decode batch prepare");
  const PagedConfig& c = s.manager.config();
  const std::size_t B = batch();
  check(tokens != 0, Status::kInvalidArgument, "decode batch prepare needs at least one token");
  check(tokens <= max_blocks_ * c.block_tokens, Status::kOutOfRange,
        "decode batch prepare: more tokens than the batch's max_tokens");
  std::size_t new_blocks = 0;
  for (std::size_t i = 0; i < B; ++i) {
    check(s.manager.contains(sequences_[i]), Status::kInvalidArgument,
          "decode batch sequence was released");
    const std::size_t len = s.manager.length(sequences_[i]);
    check(s.manager.blocks(sequences_[i]).size() >= mirrored_[i], Status::kInternal,
          "decode batch table row shrank while the sequence lived");
    check(len + tokens <= max_blocks_ * c.block_tokens, Status::kOutOfRange,
          "decode batch sequence reached the batch's max_tokens");
    new_blocks += (len + tokens + c.block_tokens - 1) / c.block_tokens -
                  (len + c.block_tokens - 1) / c.block_tokens;
  }
  check(new_blocks <= s.manager.free_block_count(), Status::kResourceExhausted,
        "decode batch prepare: the pool has too few free blocks for the step");
  reserve_step(tokens);
  DeviceGuard guard(s.device);
  if (any_call_ && last_stream_ != stream) {
    // The previous step's last call may still read the step buffers and
    // tables this step rewrites.
    hip_check(hipEventRecord(order_event_, last_stream_), "decode batch order event");
    hip_check(hipStreamWaitEvent(stream, order_event_, 0), "decode batch order wait");
  }

  const int which = next_pinned_;
  next_pinned_ ^= 1;
  hip_check(hipEventSynchronize(uploaded_[which]), "decode batch staging wait");
  auto* host = static_cast<unsigned char*>(pinned_[which].data());
  auto* lengths = reinterpret_cast<std::int32_t*>(host);
  auto* slots = reinterpret_cast<std::int64_t*>(host + align8(B * sizeof(std::int32_t)));
  auto* updates = reinterpret_cast<std::uint32_t*>(slots + B * tokens);  // host staging
  std::size_t n_updates = 0;
  for (std::size_t i = 0; i < B; ++i) {
    const AppendPlan plan = s.manager.plan_append(sequences_[i], tokens);
    s.manager.commit_append(plan);
    lengths[i] = static_cast<std::int32_t>(plan.old_length);
    host_lengths_[i] = lengths[i];
    for (std::size_t t = 0; t < tokens; ++t) {
      slots[i * tokens + t] = static_cast<std::int64_t>(plan.slot(t, c.block_tokens));
    }
    // Every entry the device row lacks: the pages this step allocated and
    // any the sequence gained outside the batch since the last step.
    const std::vector<std::uint32_t>& row = s.manager.blocks(sequences_[i]);
    for (std::size_t k = mirrored_[i]; k < row.size(); ++k) {
      updates[3 * n_updates] = static_cast<std::uint32_t>(i);
      updates[3 * n_updates + 1] = static_cast<std::uint32_t>(k);
      updates[3 * n_updates + 2] = row[k];
      mirror_[i * max_blocks_ + k] = row[k];
      ++n_updates;
    }
    mirrored_[i] = row.size();
  }
  const std::size_t used = align8(B * sizeof(std::int32_t)) + B * tokens * sizeof(std::int64_t) +
                           3 * n_updates * sizeof(std::uint32_t);
  if (tokens > 1) {
    // Longest-first order of the prefill work items: a (sequence, position
    // block) sees its history plus the chunk rows up to the block's end.
    const std::size_t H = c.kv_heads;
    const std::size_t pw = hip::prefill_position_block(q_heads_ / H);
    const std::size_t nb = (tokens + pw - 1) / pw;
    std::vector<std::pair<std::size_t, std::uint32_t>> items;
    items.reserve(B * H * nb);
    for (std::size_t i = 0; i < B; ++i) {
      for (std::size_t h = 0; h < H; ++h) {
        for (std::size_t pb = 0; pb < nb; ++pb) {
          const std::size_t work = static_cast<std::size_t>(lengths[i]) +
                                   std::min(tokens, (pb + 1) * pw);
          items.emplace_back(work, static_cast<std::uint32_t>((i * H + h) * nb + pb));
        }
      }
    }
    std::stable_sort(items.begin(), items.end(),
                     [](const auto& x, const auto& y) { return x.first > y.first; });
    auto* order = reinterpret_cast<std::uint32_t*>(host + order_offset(tokens));
    for (std::size_t n = 0; n < items.size(); ++n) order[n] = items[n].second;
    hip_check(hipMemcpyAsync(static_cast<unsigned char*>(step_.data()) + order_offset(tokens),
                             order, items.size() * sizeof(std::uint32_t), hipMemcpyHostToDevice,
                             stream),
              "decode batch order upload");
  }
  hip_check(hipMemcpyAsync(step_.data(), host, used, hipMemcpyHostToDevice, stream),
            "decode batch step upload");
  items_ = hip::decode_items(host_lengths_.data(), B, c.kv_heads, max_blocks_, pages_per_split_);
  // The updates follow the slots in the device copy of the step buffer.
  const auto* dev_updates = reinterpret_cast<const std::uint32_t*>(this->slots() + B * tokens);
  hip_check(hip::launch_table_updates(static_cast<std::uint32_t*>(tables_.data()), max_blocks_,
                                      dev_updates, n_updates, stream),
            "decode batch table update");
  // Marks the end of the step's upload: the staging copy may be reused once
  // it completes, and per-step calls on other streams wait for it.
  hip_check(hipEventRecord(uploaded_[which], stream), "decode batch event");
  prepared_event_ = which;
  prepared_stream_ = stream;
  last_stream_ = stream;
  any_call_ = true;
  prepared_releases_ = s.releases.load(std::memory_order_acquire);
  // Cascade for decode steps: the longest run of leading pages that every
  // sequence shares (same physical IDs, all full before the step) is
  // attended once for the whole batch.
  shared_pages_ = 0;
  if (tokens == 1 && pages_per_split_ == 0 && B >= kMinCascadeBatch) {
    const auto& first = s.manager.blocks(sequences_[0]);
    std::size_t shared = first.size();
    for (std::size_t i = 0; i < B && shared > 0; ++i) {
      const auto& blocks = s.manager.blocks(sequences_[i]);
      shared = std::min(shared, static_cast<std::size_t>(host_lengths_[i]) / c.block_tokens);
      std::size_t k = 0;
      while (k < shared && blocks[k] == first[k]) ++k;
      shared = k;
    }
    if (shared >= kMinCascadePages) shared_pages_ = shared;
  }
  if (shared_pages_ > 0 && side_stream_ == nullptr &&
      q_heads_ / c.kv_heads > hip::kCascadeFusedMaxGroup) {
    // Large query groups run the cascade prefix pass on this stream beside
    // the stream kernel (smaller ones launch both as one kernel).
    hip_check(hipStreamCreateWithFlags(&side_stream_, hipStreamNonBlocking), "hipStreamCreate");
    hip_check(hipEventCreateWithFlags(&fork_event_, hipEventDisableTiming), "hipEventCreate");
    hip_check(hipEventCreateWithFlags(&join_event_, hipEventDisableTiming), "hipEventCreate");
  }
  step_tokens_ = tokens;
  prepared_ = true;
}

void DecodeBatch::begin_call(hipStream_t stream, const char* op) const {
  check(prepared_, Status::kInvalidArgument, std::string(op) + " before prepare");
  CacheState& s = *state_;
  if (s.releases.load(std::memory_order_acquire) != prepared_releases_) {
    // Something was released since prepare(): the step is only valid if
    // every member still lives (their pages are the step's).
    std::scoped_lock lock(s.mutex);
    for (std::uint64_t seq : sequences_) {
      check(s.manager.contains(seq), Status::kInvalidArgument,
            std::string(op) + ": a sequence of the batch was released after prepare");
    }
    prepared_releases_ = s.releases.load(std::memory_order_acquire);
  }
  if (stream != prepared_stream_) {
    hip_check(hipStreamWaitEvent(stream, uploaded_[prepared_event_], 0),
              "decode batch stream order");
  }
  last_stream_ = stream;
}

void DecodeBatch::append_layer(std::size_t layer, const float* keys, const float* values,
                               hipStream_t stream) const {
  const PagedConfig& c = state_->manager.config();
  check(prepared_, Status::kInvalidArgument, "decode batch append before prepare");
  check(layer < c.layers, Status::kOutOfRange, "decode batch layer is out of range");
  check(keys != nullptr && values != nullptr, Status::kInvalidArgument,
        "decode batch append needs key and value rows");
  DeviceGuard guard(state_->device);
  begin_call(stream, "decode batch append");
  hip_check(hip::launch_append_slots(keys, values, state_->key_pool(layer),
                                     state_->value_pool(layer),
                                     hip::PageGeometry{c.physical_blocks, c.kv_heads,
                                                       c.block_tokens, c.head_dimension},
                                     slots(), batch(), stream, step_tokens_, state_->page_type),
            "decode batch append launch");
}

void DecodeBatch::append_all_layers(const float* keys, const float* values,
                                    hipStream_t stream) const {
  const PagedConfig& c = state_->manager.config();
  check(prepared_, Status::kInvalidArgument, "decode batch append before prepare");
  check(keys != nullptr && values != nullptr, Status::kInvalidArgument,
        "decode batch append needs key and value rows");
  DeviceGuard guard(state_->device);
  begin_call(stream, "decode batch append");
  hip_check(hip::launch_append_slots(keys, values, state_->key_pool(0), state_->value_pool(0),
                                     hip::PageGeometry{c.physical_blocks, c.kv_heads,
                                                       c.block_tokens, c.head_dimension},
                                     slots(), batch(), stream, step_tokens_, state_->page_type,
                                     c.layers, state_->layer_stride()),
            "decode batch append launch");
}

void DecodeBatch::rope(float* query, float* key, const float* cosine, const float* sine,
                       std::size_t cache_rows, hipStream_t stream) const {
  const PagedConfig& c = state_->manager.config();
  check(prepared_, Status::kInvalidArgument, "decode batch rope before prepare");
  check(step_tokens_ == 1, Status::kInvalidArgument,
        "decode batch rope needs a one-token step (positions of chunk rows differ)");
  check(query != nullptr && key != nullptr && cosine != nullptr && sine != nullptr,
        Status::kInvalidArgument, "decode batch rope needs query, key and the rope tables");
  check(cache_rows != 0, Status::kInvalidArgument, "decode batch rope tables have no rows");
  DeviceGuard guard(state_->device);
  begin_call(stream, "decode batch rope");
  hip_check(hip::launch_rope(hip::RopeTensor{query, query, q_heads_},
                             hip::RopeTensor{key, key, c.kv_heads}, batch(), c.head_dimension,
                             cosine, sine, cache_rows, lengths(), stream),
            "decode batch rope launch");
}

void DecodeBatch::append_attention_layer(std::size_t layer, const float* query,
                                         const float* keys, const float* values, float* out,
                                         hipStream_t stream) const {
  if (pages_per_split_ != 0) {
    append_layer(layer, keys, values, stream);
    attention_layer(layer, query, keys, values, out, stream);
    return;
  }
  attention_layer(layer, query, keys, values, out, stream, true);
}

void DecodeBatch::attention_layer(std::size_t layer, const float* query, const float* tail_key,
                                  const float* tail_value, float* out, hipStream_t stream,
                                  bool fused_append) const {
  const PagedConfig& c = state_->manager.config();
  check(prepared_, Status::kInvalidArgument, "decode batch attention before prepare");
  check(step_tokens_ == 1, Status::kInvalidArgument,
        "decode batch attention needs a one-token step (use prefill for chunks)");
  check(layer < c.layers, Status::kOutOfRange, "decode batch layer is out of range");
  check(query != nullptr && tail_key != nullptr && tail_value != nullptr && out != nullptr,
        Status::kInvalidArgument, "decode batch attention needs query, tail and output");
  hip::DecodeArgs a{};
  a.query = query;
  a.key_pool = state_->key_pool(layer);
  a.value_pool = state_->value_pool(layer);
  a.tables = tables();
  a.lengths = lengths();
  a.tail_key = tail_key;
  a.tail_value = tail_value;
  a.out = out;
  a.workspace = workspace_.data();
  a.batch = batch();
  a.q_heads = q_heads_;
  a.kv_heads = c.kv_heads;
  a.max_blocks = max_blocks_;
  a.physical_blocks = c.physical_blocks;
  a.pages_per_split = pages_per_split_;
  a.items = items_;
  a.between_event = between_event_;
  a.shared_pages = shared_pages_;
  a.page_type = state_->page_type;
  a.side_stream = side_stream_;
  a.fork_event = fork_event_;
  a.join_event = join_event_;
  if (fused_append) {
    a.append_slots = slots();
    a.append_key_pool = state_->key_pool(layer);
    a.append_value_pool = state_->value_pool(layer);
  }
  DeviceGuard guard(state_->device);
  begin_call(stream, "decode batch attention");
  hip_check(hip::launch_decode(a, stream), "decode batch attention launch");
}

void DecodeBatch::prefill_layer(std::size_t layer, const float* query, const float* chunk_key,
                                const float* chunk_value, float* out, hipStream_t stream) const {
  const PagedConfig& c = state_->manager.config();
  check(prepared_, Status::kInvalidArgument, "decode batch prefill before prepare");
  check(layer < c.layers, Status::kOutOfRange, "decode batch layer is out of range");
  check(query != nullptr && chunk_key != nullptr && chunk_value != nullptr && out != nullptr,
        Status::kInvalidArgument, "decode batch prefill needs query, chunk and output");
  hip::PrefillArgs a{};
  a.query = query;
  a.key_pool = state_->key_pool(layer);
  a.value_pool = state_->value_pool(layer);
  a.tables = tables();
  a.lengths = lengths();
  a.chunk_key = chunk_key;
  a.chunk_value = chunk_value;
  a.out = out;
  a.batch = batch();
  a.q_heads = q_heads_;
  a.kv_heads = c.kv_heads;
  a.tokens = step_tokens_;
  a.max_blocks = max_blocks_;
  a.physical_blocks = c.physical_blocks;
  a.page_type = state_->page_type;
  if (step_tokens_ > 1) {
    a.order = reinterpret_cast<const std::uint32_t*>(
        static_cast<const unsigned char*>(step_.data()) + order_offset(step_tokens_));
  }
  a.redo = reinterpret_cast<std::uint32_t*>(
      static_cast<unsigned char*>(step_.data()) + order_offset(step_tokens_) +
      prefill_items(step_tokens_) * sizeof(std::uint32_t));
  DeviceGuard guard(state_->device);
  begin_call(stream, "decode batch prefill");
  hip_check(hip::launch_prefill(a, stream), "decode batch prefill launch");
}

}  // namespace helix
