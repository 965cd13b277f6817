/* C++ mirror of the reference's paged-KV and paged-attention API over the
 * C ABI in helix_paged.h (header-only, C++20).
 *
 * The classes and functions keep the reference's names, argument meaning and
 * error behaviour, so code written against the reference's CUDA path reads
 * the same here:
 *
 *   helix::kv_cache::CudaPagedKvCache          -> helix_amd::kv_cache::HipPagedKvCache
 *       (include/helix/kv_cache/cuda_paged.hpp:47-108)
 *   helix::kv_cache::CudaPagedSequenceHandle   -> helix_amd::kv_cache::HipPagedSequenceHandle
 *       (include/helix/kv_cache/cuda_paged.hpp:18-42)
 *   helix::kv_cache::cuda::PagedBlockTable     -> helix_amd::kv_cache::hip::PagedBlockTable
 *       (include/helix/kv_cache/cuda_block_table.hpp:14-50)
 *   helix::attention::cuda::paged_*            -> helix_amd::attention::hip::paged_*
 *       (include/helix/attention/cuda_paged.hpp:15-80)
 *   helix::kv_cache::PagedPrefixCache          -> helix_amd::kv_cache::HipPagedPrefixCache
 *       (include/helix/kv_cache/prefix.hpp:77-113), over the device cache
 *   helix::Error / helix::ErrorCode            -> helix_amd::Error / helix_amd::ErrorCode
 *       (include/helix/core/error.hpp:10-38)
 *
 * with `Cuda*` aliases and `cuda` namespace aliases beside the HIP names.
 * Tensors are this header's own small fp32-centric Tensor (the reference's
 * Tensor is not part of the boundary): device tensors own HIP memory or
 * borrow it (tensors a DecodeView hands out keep the cache's pools alive, as
 * the reference's do).
 *
 * Every call validates tensor dtype, device and rank here and passes plain
 * pointers and sizes to the C ABI, which validates geometry, table contents
 * and aliasing before any launch; a non-zero status becomes helix_amd::Error
 * with the matching ErrorCode and the library's message.  Kernels run
 * asynchronously on the caller's stream; the allocating forms synchronise
 * before returning (include/helix/attention/cuda_paged.hpp:62-80).
 *
 * Extensions beyond the reference's CUDA API (each also in helix_paged.h):
 * fork_sequence with copy-on-write, append_layer_major, copy_layer_out,
 * bf16 pages, and DecodeBatch, the batched decode / chunked-prefill driver.
 *
 * Link with -lhelix_paged -lamdhip64; compile with -D__HIP_PLATFORM_AMD__
 * when the compiler is not hipcc. */
#ifndef HELIX_PAGED_HPP
#define HELIX_PAGED_HPP

#include "helix_paged.h"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace helix_amd {

// ------------------------------------------------------------------ errors --

/// include/helix/core/error.hpp:10-17; the C status is this value plus one.
enum class ErrorCode {
  kInvalidArgument,
  kOutOfRange,
  kUnsupported,
  kResourceExhausted,
  kRuntime,
  kInternal,
};

[[nodiscard]] inline std::string_view error_code_name(ErrorCode code) noexcept {
  switch (code) {
    case ErrorCode::kInvalidArgument: return "InvalidArgument";
    case ErrorCode::kOutOfRange: return "OutOfRange";
    case ErrorCode::kUnsupported: return "Unsupported";
    case ErrorCode::kResourceExhausted: return "ResourceExhausted";
    case ErrorCode::kRuntime: return "Runtime";
    case ErrorCode::kInternal: return "Internal";
  }
  return "Unknown";
}

/// include/helix/core/error.hpp:19-38 (without the source location).
class Error final : public std::runtime_error {
 public:
  Error(ErrorCode code, std::string message)
      : std::runtime_error(std::string(error_code_name(code)) + ": " + message),
        code_(code),
        message_(std::move(message)) {}
  [[nodiscard]] ErrorCode code() const noexcept { return code_; }
  [[nodiscard]] const std::string& message() const noexcept { return message_; }

 private:
  ErrorCode code_;
  std::string message_;
};

[[noreturn]] inline void throw_error(ErrorCode code, std::string message) {
  throw Error(code, std::move(message));
}

namespace detail {

/// Status from the C ABI -> Error (helix_last_error() carries the message).
inline void check(int status) {
  if (status == HELIX_OK) return;
  const ErrorCode code = status >= HELIX_INVALID_ARGUMENT && status <= HELIX_INTERNAL
                             ? static_cast<ErrorCode>(status - 1)
                             : ErrorCode::kInternal;
  throw_error(code, helix_last_error());
}

inline void require(bool condition, ErrorCode code, const char* message) {
  if (!condition) throw_error(code, message);
}

inline void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) {
    throw_error(ErrorCode::kRuntime, std::string(what) + ": " + hipGetErrorString(status));
  }
}

}  // namespace detail

// ------------------------------------------------------------------ tensor --

enum class DType { kFloat32, kBFloat16, kInt32, kInt64, kUInt32, kFp8E4M3 };

[[nodiscard]] constexpr std::size_t dtype_size(DType d) noexcept {
  return d == DType::kFp8E4M3 ? 1 : d == DType::kBFloat16 ? 2 : (d == DType::kInt64 ? 8 : 4);
}

struct Device {
  enum class Kind { kCpu, kGpu };
  Kind kind = Kind::kCpu;
  int index = 0;
  [[nodiscard]] static constexpr Device cpu() noexcept { return {Kind::kCpu, 0}; }
  [[nodiscard]] static constexpr Device gpu(int index) noexcept { return {Kind::kGpu, index}; }
  /// The reference's spelling of a GPU device.
  [[nodiscard]] static constexpr Device cuda(int index) noexcept { return gpu(index); }
  [[nodiscard]] constexpr bool is_gpu() const noexcept { return kind == Kind::kGpu; }
  friend constexpr bool operator==(const Device&, const Device&) = default;
};

using Dimension = std::int64_t;
using Shape = std::vector<Dimension>;

[[nodiscard]] inline std::size_t shape_numel(const Shape& shape) {
  std::size_t n = 1;
  for (Dimension d : shape) {
    detail::require(d >= 0, ErrorCode::kInvalidArgument, "Tensor: negative dimension");
    n *= static_cast<std::size_t>(d);
  }
  return n;
}

/// A dense row-major tensor in host or device memory.  Storage is shared:
/// reshape() and copies of a Tensor alias the same bytes.
class Tensor {
 public:
  Tensor() = default;

  [[nodiscard]] static Tensor empty(Shape shape, DType dtype = DType::kFloat32,
                                    Device device = Device::cpu()) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.device_ = device;
    const std::size_t bytes = t.nbytes();
    if (device.is_gpu()) {
      int current = 0;
      detail::check_hip(hipGetDevice(&current), "hipGetDevice");
      detail::check_hip(hipSetDevice(device.index), "hipSetDevice");
      void* p = nullptr;
      const hipError_t rc = hipMalloc(&p, bytes == 0 ? 1 : bytes);
      (void)hipSetDevice(current);
      detail::check_hip(rc, "hipMalloc");
      t.storage_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
    } else {
      t.storage_ = std::shared_ptr<void>(::operator new(bytes == 0 ? 1 : bytes),
                                         [](void* q) { ::operator delete(q); });
    }
    t.data_ = t.storage_.get();
    return t;
  }

  [[nodiscard]] static Tensor zeros(Shape shape, DType dtype = DType::kFloat32,
                                    Device device = Device::cpu()) {
    Tensor t = empty(std::move(shape), dtype, device);
    if (device.is_gpu()) {
      detail::check_hip(hipMemset(t.data_, 0, t.nbytes()), "hipMemset");
    } else if (t.nbytes() != 0) {
      std::memset(t.data_, 0, t.nbytes());
    }
    return t;
  }

  /// float32 values, host first then copied to `device`.
  [[nodiscard]] static Tensor from_values(Shape shape, std::span<const float> values,
                                          Device device = Device::cpu()) {
    Tensor host = empty(std::move(shape), DType::kFloat32, Device::cpu());
    detail::require(values.size() == host.numel(), ErrorCode::kInvalidArgument,
                    "Tensor::from_values: value count must match the shape");
    if (!values.empty()) std::memcpy(host.data_, values.data(), host.nbytes());
    return device.is_gpu() ? host.to(device) : host;
  }
  template <class Range>
  [[nodiscard]] static Tensor from_values(Shape shape, const Range& values,
                                          Device device = Device::cpu()) {
    return from_values(std::move(shape), std::span<const float>(values), device);
  }

  /// Wrap memory the caller owns (`owner`, when given, is kept alive).
  [[nodiscard]] static Tensor borrow(void* data, Shape shape, DType dtype, Device device,
                                     std::shared_ptr<void> owner = {}) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.device_ = device;
    t.data_ = data;
    t.storage_ = std::move(owner);
    return t;
  }

  /// Synchronous copy to `device` (hipMemcpy orders after the null stream).
  [[nodiscard]] Tensor to(Device device) const {
    Tensor out = empty(shape_, dtype_, device);
    if (nbytes() == 0) return out;
    const hipMemcpyKind kind =
        device_.is_gpu() ? (device.is_gpu() ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost)
                         : (device.is_gpu() ? hipMemcpyHostToDevice : hipMemcpyHostToHost);
    detail::check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
    detail::check_hip(hipMemcpy(out.data_, data_, nbytes(), kind), "hipMemcpy");
    return out;
  }

  [[nodiscard]] Tensor reshape(Shape shape) const {
    detail::require(shape_numel(shape) == numel(), ErrorCode::kInvalidArgument,
                    "Tensor::reshape: element count must not change");
    Tensor t = *this;
    t.shape_ = std::move(shape);
    return t;
  }

  [[nodiscard]] const Shape& shape() const noexcept { return shape_; }
  [[nodiscard]] std::size_t rank() const noexcept { return shape_.size(); }
  [[nodiscard]] DType dtype() const noexcept { return dtype_; }
  [[nodiscard]] Device device() const noexcept { return device_; }
  [[nodiscard]] std::size_t numel() const { return shape_numel(shape_); }
  [[nodiscard]] std::size_t nbytes() const { return numel() * dtype_size(dtype_); }
  [[nodiscard]] bool defined() const noexcept { return data_ != nullptr || !shape_.empty(); }
  template <class T>
  [[nodiscard]] T* data() const noexcept {
    return static_cast<T*>(data_);
  }
  template <class T>
  [[nodiscard]] const T* data_as() const noexcept {
    return static_cast<const T*>(data_);
  }
  [[nodiscard]] void* raw() const noexcept { return data_; }

 private:
  std::shared_ptr<void> storage_;
  void* data_ = nullptr;
  Shape shape_;
  DType dtype_ = DType::kFloat32;
  Device device_ = Device::cpu();
};

// ----------------------------------------------------------------- runtime --

namespace hip {

[[nodiscard]] inline bool runtime_available() noexcept {
  int count = 0;
  return hipGetDeviceCount(&count) == hipSuccess && count > 0;
}

inline void set_device(int index) { detail::check_hip(hipSetDevice(index), "hipSetDevice"); }

/// An owned HIP stream at the default priority (helix::cuda::Stream).  A
/// moved-from stream is invalid and every call that takes it throws.
class Stream {
 public:
  Stream() { detail::check_hip(hipStreamCreate(&stream_), "hipStreamCreate"); }
  ~Stream() {
    if (stream_ != nullptr) (void)hipStreamDestroy(stream_);
  }
  Stream(const Stream&) = delete;
  Stream& operator=(const Stream&) = delete;
  Stream(Stream&& other) noexcept : stream_(std::exchange(other.stream_, nullptr)) {}
  Stream& operator=(Stream&& other) noexcept {
    if (this != &other) {
      if (stream_ != nullptr) (void)hipStreamDestroy(stream_);
      stream_ = std::exchange(other.stream_, nullptr);
    }
    return *this;
  }
  [[nodiscard]] bool valid() const noexcept { return stream_ != nullptr; }
  [[nodiscard]] hipStream_t native() const {
    detail::require(stream_ != nullptr, ErrorCode::kInvalidArgument,
                    "Stream: the stream is not valid (moved from)");
    return stream_;
  }
  void synchronize() const { detail::check_hip(hipStreamSynchronize(native()), "hipStreamSynchronize"); }

 private:
  hipStream_t stream_ = nullptr;
};

}  // namespace hip
namespace cuda = hip;

namespace detail {

inline void require_float_on(const Tensor& t, int device, std::size_t rank, const char* what) {
  if (t.dtype() != DType::kFloat32 || !t.device().is_gpu() || t.device().index != device ||
      t.rank() != rank) {
    throw_error(ErrorCode::kInvalidArgument,
                std::string(what) + ": expected a float32 tensor of rank " + std::to_string(rank) +
                    " on GPU " + std::to_string(device));
  }
}

inline std::size_t dim(const Tensor& t, std::size_t i) {
  return static_cast<std::size_t>(t.shape()[i]);
}

inline int current_device() {
  int d = 0;
  check_hip(hipGetDevice(&d), "hipGetDevice");
  return d;
}

}  // namespace detail

// --------------------------------------------------------------- kv cache --

namespace kv_cache {

/// include/helix/kv_cache/paged.hpp:60-66.
struct PagedKvCacheConfig {
  std::size_t layers = 0;
  std::size_t kv_heads = 0;
  std::size_t head_dimension = 0;
  std::size_t block_tokens = 0;
  std::size_t physical_blocks = 0;
};

/// include/helix/kv_cache/paged.hpp:68-107.
struct PagedKvCacheStats {
  std::size_t bytes_reserved = 0;
  std::size_t bytes_used = 0;
  std::size_t bytes_free = 0;
  std::size_t peak_bytes_used = 0;
  std::size_t total_blocks = 0;
  std::size_t used_blocks = 0;
  std::size_t free_blocks = 0;
  std::size_t active_sequence_count = 0;
  std::size_t active_tokens = 0;
  std::size_t resident_tokens = 0;
  std::size_t allocated_token_slots = 0;
  std::size_t block_reference_count = 0;
  std::size_t shared_blocks = 0;
  std::uint64_t sequence_create_count = 0;
  std::uint64_t sequence_fork_count = 0;
  std::uint64_t append_count = 0;
  std::uint64_t release_count = 0;
  std::uint64_t block_allocation_count = 0;
  std::uint64_t block_reuse_count = 0;

  [[nodiscard]] std::size_t unused_token_slots() const noexcept {
    return allocated_token_slots - resident_tokens;
  }
  [[nodiscard]] std::size_t shared_token_references() const noexcept {
    return active_tokens - resident_tokens;
  }
  [[nodiscard]] double token_slot_utilization() const noexcept {
    return allocated_token_slots == 0
               ? 0.0
               : static_cast<double>(resident_tokens) / static_cast<double>(allocated_token_slots);
  }
};

/// Page storage type (extension: bf16 pages halve HBM bytes per token, fp8
/// E4M3 pages quarter them; fp8 scales as Fp8Scales, 1 and 1 by default).
enum class PageDType {
  kFloat32 = HELIX_PAGE_F32,
  kBFloat16 = HELIX_PAGE_BF16,
  kFp8E4M3 = HELIX_PAGE_FP8_E4M3
};
/// The key and value scales of an fp8 cache: a page element is the E4M3
/// code of x / scale (nearest even, saturating at +-448), worth
/// decode(code) * scale.
struct Fp8Scales {
  float key = 1.0F;
  float value = 1.0F;
};

class HipPagedKvCache;
class HipPagedPrefixCache;
class DecodeBatch;

/// include/helix/kv_cache/cuda_paged.hpp:18-42: a non-owning {sequence id,
/// cache id} pair; id 0 is the empty handle.
class HipPagedSequenceHandle final {
 public:
  HipPagedSequenceHandle() = default;
  [[nodiscard]] explicit operator bool() const noexcept { return sequence_id_ != 0; }
  [[nodiscard]] std::uint64_t id() const noexcept { return sequence_id_; }
  [[nodiscard]] std::uint64_t cache_id() const noexcept { return cache_id_; }
  /// The C ABI's form of the handle.
  [[nodiscard]] helix_sequence native() const noexcept { return {sequence_id_, cache_id_}; }
  friend bool operator==(const HipPagedSequenceHandle&, const HipPagedSequenceHandle&) = default;

 private:
  friend class HipPagedKvCache;
  friend class HipPagedPrefixCache;
  HipPagedSequenceHandle(std::uint64_t sequence_id, std::uint64_t cache_id) noexcept
      : sequence_id_(sequence_id), cache_id_(cache_id) {}
  explicit HipPagedSequenceHandle(helix_sequence s) noexcept
      : sequence_id_(s.id), cache_id_(s.cache_id) {}

  std::uint64_t sequence_id_ = 0;
  std::uint64_t cache_id_ = 0;
};

namespace hip {

using Stream = helix_amd::hip::Stream;

/// include/helix/kv_cache/cuda_block_table.hpp:14-50: a device copy of a
/// logical -> physical page list, validated against the pool capacity on
/// construction.  An empty list is valid and has data() == nullptr.  Tables
/// a DecodeView hands out borrow the view's device copy.
class PagedBlockTable final {
 public:
  PagedBlockTable(std::span<const std::uint32_t> physical_blocks, std::size_t physical_block_count,
                  int device_index)
      : logical_block_count_(physical_blocks.size()),
        physical_block_count_(physical_block_count),
        device_index_(device_index) {
    helix_block_table* t = nullptr;
    detail::check(helix_block_table_create(physical_blocks.data(), physical_blocks.size(),
                                           physical_block_count, device_index, &t));
    owned_ = t;
    data_ = helix_block_table_data(t);
    valid_ = true;
  }
  ~PagedBlockTable() {
    if (owned_ != nullptr) helix_block_table_destroy(owned_);
  }
  PagedBlockTable(const PagedBlockTable&) = delete;
  PagedBlockTable& operator=(const PagedBlockTable&) = delete;
  PagedBlockTable(PagedBlockTable&& o) noexcept
      : owned_(std::exchange(o.owned_, nullptr)),
        data_(std::exchange(o.data_, nullptr)),
        logical_block_count_(std::exchange(o.logical_block_count_, 0)),
        physical_block_count_(std::exchange(o.physical_block_count_, 0)),
        device_index_(std::exchange(o.device_index_, -1)),
        valid_(std::exchange(o.valid_, false)) {}
  PagedBlockTable& operator=(PagedBlockTable&& o) noexcept {
    if (this != &o) {
      if (owned_ != nullptr) helix_block_table_destroy(owned_);
      owned_ = std::exchange(o.owned_, nullptr);
      data_ = std::exchange(o.data_, nullptr);
      logical_block_count_ = std::exchange(o.logical_block_count_, 0);
      physical_block_count_ = std::exchange(o.physical_block_count_, 0);
      device_index_ = std::exchange(o.device_index_, -1);
      valid_ = std::exchange(o.valid_, false);
    }
    return *this;
  }

  [[nodiscard]] bool valid() const noexcept { return valid_; }
  [[nodiscard]] const std::uint32_t* data() const noexcept { return data_; }
  [[nodiscard]] std::size_t logical_block_count() const noexcept { return logical_block_count_; }
  [[nodiscard]] std::size_t physical_block_count() const noexcept { return physical_block_count_; }
  [[nodiscard]] std::size_t size_bytes() const noexcept {
    return logical_block_count_ * sizeof(std::uint32_t);
  }
  [[nodiscard]] int device_index() const noexcept { return device_index_; }

 private:
  friend class kv_cache::HipPagedKvCache;
  PagedBlockTable() = default;
  static PagedBlockTable borrowed(const std::uint32_t* device_table, std::size_t logical,
                                  std::size_t physical, int device) {
    PagedBlockTable t;
    t.data_ = logical == 0 ? nullptr : device_table;
    t.logical_block_count_ = logical;
    t.physical_block_count_ = physical;
    t.device_index_ = device;
    t.valid_ = true;
    return t;
  }

  helix_block_table* owned_ = nullptr;
  const std::uint32_t* data_ = nullptr;
  std::size_t logical_block_count_ = 0;
  std::size_t physical_block_count_ = 0;
  int device_index_ = -1;
  bool valid_ = false;
};

}  // namespace hip
namespace cuda = hip;

/// include/helix/kv_cache/cuda_paged.hpp:47-108: the device paged KV pool.
/// One slab holds every layer's K and V pools, each [physical_blocks,
/// kv_heads, block_tokens, head_dimension]; pages come from a FIFO free list
/// and are reference counted.  Not copyable or movable; DecodeViews keep the
/// pools alive after the cache object is gone.
class HipPagedKvCache final {
  struct Impl {
    helix_paged_cache* cache = nullptr;
    PagedKvCacheConfig config;
    int device = 0;
    std::size_t bytes_per_token = 0, block_bytes = 0, token_capacity = 0;
    ~Impl() {
      if (cache != nullptr) helix_paged_cache_destroy(cache);
    }
  };

 public:
  /// include/helix/kv_cache/cuda_paged.hpp:57-87: a read lease on one
  /// sequence.  While it lives, append and release on the cache wait; the
  /// pool tensors and the device block table it hands out stay valid.
  class DecodeView final {
   public:
    ~DecodeView() { reset(); }
    DecodeView(const DecodeView&) = delete;
    DecodeView& operator=(const DecodeView&) = delete;
    DecodeView(DecodeView&& o) noexcept
        : cache_(std::move(o.cache_)),
          view_(std::exchange(o.view_, nullptr)),
          keys_(std::move(o.keys_)),
          values_(std::move(o.values_)),
          blocks_(std::move(o.blocks_)),
          table_(std::move(o.table_)),
          length_(o.length_) {}
    DecodeView& operator=(DecodeView&& o) noexcept {
      if (this != &o) {
        reset();
        cache_ = std::move(o.cache_);
        view_ = std::exchange(o.view_, nullptr);
        keys_ = std::move(o.keys_);
        values_ = std::move(o.values_);
        blocks_ = std::move(o.blocks_);
        table_ = std::move(o.table_);
        length_ = o.length_;
      }
      return *this;
    }

    [[nodiscard]] std::size_t length() const {
      require_valid("length");
      return length_;
    }
    [[nodiscard]] std::span<const std::uint32_t> physical_blocks() const {
      require_valid("physical_blocks");
      return blocks_;
    }
    [[nodiscard]] std::span<const Tensor> layer_key_blocks() const {
      require_valid("layer_key_blocks");
      return keys_;
    }
    [[nodiscard]] std::span<const Tensor> layer_value_blocks() const {
      require_valid("layer_value_blocks");
      return values_;
    }
    [[nodiscard]] const hip::PagedBlockTable& block_table() const {
      require_valid("block_table");
      return *table_;
    }
    /// include/helix/kv_cache/cuda_paged.hpp:70: a consumer whose kernels on
    /// these pages failed quarantines the table; the cache turns unhealthy.
    void poison_after_consumer_failure() noexcept {
      if (view_ != nullptr) helix_decode_view_poison(view_);
      reset();
    }

   private:
    friend class HipPagedKvCache;
    DecodeView() = default;
    void require_valid(const char* operation) const {
      if (view_ == nullptr) {
        throw_error(ErrorCode::kInvalidArgument,
                    std::string("DecodeView::") + operation + ": the view is no longer valid");
      }
    }
    void reset() noexcept {
      keys_.clear();
      values_.clear();
      blocks_.clear();
      table_.reset();
      if (view_ != nullptr) helix_decode_view_release(std::exchange(view_, nullptr));
      cache_.reset();
    }

    std::shared_ptr<Impl> cache_;
    helix_decode_view* view_ = nullptr;
    std::vector<Tensor> keys_, values_;
    std::vector<std::uint32_t> blocks_;
    std::optional<hip::PagedBlockTable> table_;
    std::size_t length_ = 0;
  };

  explicit HipPagedKvCache(PagedKvCacheConfig config, int device_index = 0,
                           PageDType pages = PageDType::kFloat32, Fp8Scales scales = {})
      : impl_(std::make_shared<Impl>()) {
    detail::require(device_index >= 0, ErrorCode::kInvalidArgument,
                    "HipPagedKvCache: device index must be non-negative");
    detail::require(pages == PageDType::kFp8E4M3 || (scales.key == 1.0F && scales.value == 1.0F),
                    ErrorCode::kInvalidArgument,
                    "HipPagedKvCache: fp8 scales apply to fp8 pages only");
    const helix_paged_config c{config.layers, config.kv_heads, config.head_dimension,
                               config.block_tokens, config.physical_blocks};
    if (pages == PageDType::kFp8E4M3) {
      detail::check(helix_paged_cache_create_fp8(&c, device_index, scales.key, scales.value,
                                                 &impl_->cache));
    } else {
      detail::check(helix_paged_cache_create_typed(&c, device_index, static_cast<int>(pages),
                                                   &impl_->cache));
    }
    impl_->config = config;
    impl_->device = device_index;
    detail::check(helix_paged_cache_geometry(impl_->cache, &impl_->bytes_per_token,
                                             &impl_->block_bytes, &impl_->token_capacity));
  }
  ~HipPagedKvCache() = default;
  HipPagedKvCache(const HipPagedKvCache&) = delete;
  HipPagedKvCache& operator=(const HipPagedKvCache&) = delete;
  HipPagedKvCache(HipPagedKvCache&&) = delete;
  HipPagedKvCache& operator=(HipPagedKvCache&&) = delete;

  [[nodiscard]] HipPagedSequenceHandle create_sequence() {
    helix_sequence s{};
    detail::check(helix_paged_cache_create_sequence(impl_->cache, &s));
    return HipPagedSequenceHandle(s);
  }

  /// One token's K and V, each [layers, kv_heads, head_dimension] float32 on
  /// the cache's device: allocates a page when the last one is full and
  /// writes every (layer, head) row in one launch on `stream`
  /// (src/kv_cache/cuda_paged.cpp:491-611).
  void append(const HipPagedSequenceHandle& sequence, const Tensor& token_keys,
              const Tensor& token_values, const hip::Stream& stream) {
    const auto& c = impl_->config;
    check_rows(token_keys, "append keys", {c.layers, c.kv_heads, c.head_dimension});
    check_rows(token_values, "append values", {c.layers, c.kv_heads, c.head_dimension});
    detail::check(helix_paged_cache_append(impl_->cache, sequence.native(),
                                           token_keys.data_as<float>(),
                                           token_values.data_as<float>(), stream.native()));
  }

  /// Bulk append of `tokens` tokens per layer from [kv_heads, tokens,
  /// head_dimension] tensors (PagedKvCache::append_layer_major,
  /// src/kv_cache/paged.cpp:721-871), transactional.
  void append_layer_major(const HipPagedSequenceHandle& sequence,
                          std::span<const Tensor> layer_keys, std::span<const Tensor> layer_values,
                          const hip::Stream& stream) {
    const auto& c = impl_->config;
    detail::require(layer_keys.size() == c.layers && layer_values.size() == c.layers,
                    ErrorCode::kInvalidArgument,
                    "append_layer_major: one key and one value tensor per layer");
    const std::size_t tokens = layer_keys.empty() || layer_keys[0].rank() != 3
                                   ? 0
                                   : detail::dim(layer_keys[0], 1);
    std::vector<const float*> k(c.layers), v(c.layers);
    for (std::size_t l = 0; l < c.layers; ++l) {
      check_rows(layer_keys[l], "append_layer_major keys", {c.kv_heads, tokens, c.head_dimension});
      check_rows(layer_values[l], "append_layer_major values",
                 {c.kv_heads, tokens, c.head_dimension});
      k[l] = layer_keys[l].data_as<float>();
      v[l] = layer_values[l].data_as<float>();
    }
    detail::check(helix_paged_cache_append_layer_major(impl_->cache, sequence.native(), k.data(),
                                                       v.data(), tokens, stream.native()));
  }

  /// Fork a sequence sharing the first `prefix_tokens` tokens.  Without
  /// copy-on-write the prefix must be page aligned (the reference's rule,
  /// src/kv_cache/paged.cpp:544-545); with it, the partial last page is
  /// copied into a fresh page on `stream`.
  [[nodiscard]] HipPagedSequenceHandle fork_sequence(const HipPagedSequenceHandle& source,
                                                     std::size_t prefix_tokens,
                                                     bool allow_copy_on_write,
                                                     const hip::Stream& stream) {
    helix_sequence s{};
    detail::check(helix_paged_cache_fork_sequence(impl_->cache, source.native(), prefix_tokens,
                                                  allow_copy_on_write ? 1 : 0, stream.native(),
                                                  &s));
    return HipPagedSequenceHandle(s);
  }

  void release_sequence(const HipPagedSequenceHandle& sequence) {
    detail::check(helix_paged_cache_release_sequence(impl_->cache, sequence.native()));
  }

  /// Gather one layer of a sequence into compact [kv_heads, length,
  /// head_dimension] tensors (copy_layer_out, src/kv_cache/paged.cpp:873-950).
  void copy_layer_out(const HipPagedSequenceHandle& sequence, std::size_t layer, Tensor& keys_out,
                      Tensor& values_out, const hip::Stream& stream) {
    const auto& c = impl_->config;
    const std::size_t n = length(sequence);
    check_rows(keys_out, "copy_layer_out keys", {c.kv_heads, n, c.head_dimension});
    check_rows(values_out, "copy_layer_out values", {c.kv_heads, n, c.head_dimension});
    detail::check(helix_paged_cache_copy_layer_out(impl_->cache, sequence.native(), layer,
                                                   keys_out.data<float>(),
                                                   values_out.data<float>(), stream.native()));
  }

  [[nodiscard]] DecodeView read_sequence(const HipPagedSequenceHandle& sequence) const {
    DecodeView v;
    helix_decode_view* raw = nullptr;
    detail::check(helix_paged_cache_read_sequence(impl_->cache, sequence.native(), &raw));
    v.view_ = raw;  // released by v's destructor from here on
    v.cache_ = impl_;
    detail::check(helix_decode_view_length(raw, &v.length_));
    const std::uint32_t* blocks = nullptr;
    std::size_t count = 0;
    detail::check(helix_decode_view_physical_blocks(raw, &blocks, &count));
    v.blocks_.assign(blocks, blocks + count);
    const std::uint32_t* device_table = nullptr;
    detail::check(helix_decode_view_block_table(raw, &device_table));
    const auto& c = impl_->config;
    v.table_.emplace(hip::PagedBlockTable::borrowed(device_table, count, c.physical_blocks,
                                                    impl_->device));
    const Shape pool{static_cast<Dimension>(c.physical_blocks), static_cast<Dimension>(c.kv_heads),
                     static_cast<Dimension>(c.block_tokens),
                     static_cast<Dimension>(c.head_dimension)};
    int dtype = HELIX_PAGE_F32;
    detail::check(helix_paged_cache_page_dtype(impl_->cache, &dtype));
    const DType element = dtype == HELIX_PAGE_BF16      ? DType::kBFloat16
                          : dtype == HELIX_PAGE_FP8_E4M3 ? DType::kFp8E4M3
                                                         : DType::kFloat32;
    for (std::size_t l = 0; l < c.layers; ++l) {
      float* k = nullptr;
      float* vv = nullptr;
      detail::check(helix_decode_view_layer_pools(raw, l, &k, &vv));
      v.keys_.push_back(Tensor::borrow(k, pool, element, Device::gpu(impl_->device), impl_));
      v.values_.push_back(Tensor::borrow(vv, pool, element, Device::gpu(impl_->device), impl_));
    }
    return v;
  }

  [[nodiscard]] bool is_healthy() const {
    int ok = 0;
    detail::check(helix_paged_cache_is_healthy(impl_->cache, &ok));
    return ok != 0;
  }
  [[nodiscard]] bool contains(const HipPagedSequenceHandle& sequence) const {
    int out = 0;
    detail::check(helix_paged_cache_contains(impl_->cache, sequence.native(), &out));
    return out != 0;
  }
  [[nodiscard]] std::size_t length(const HipPagedSequenceHandle& sequence) const {
    std::size_t out = 0;
    detail::check(helix_paged_cache_length(impl_->cache, sequence.native(), &out));
    return out;
  }
  /// The sequence's logical -> physical page list (a host snapshot).
  [[nodiscard]] std::vector<std::uint32_t> block_table(const HipPagedSequenceHandle& s) const {
    std::vector<std::uint32_t> out(impl_->config.physical_blocks);
    std::size_t count = 0;
    detail::check(helix_paged_cache_block_table(impl_->cache, s.native(), out.data(), out.size(),
                                                &count));
    out.resize(count);
    return out;
  }
  [[nodiscard]] PagedKvCacheStats stats() const {
    helix_paged_stats s{};
    detail::check(helix_paged_cache_stats(impl_->cache, &s));
    PagedKvCacheStats r;
    r.bytes_reserved = s.bytes_reserved;
    r.bytes_used = s.bytes_used;
    r.bytes_free = s.bytes_free;
    r.peak_bytes_used = s.peak_bytes_used;
    r.total_blocks = s.total_blocks;
    r.used_blocks = s.used_blocks;
    r.free_blocks = s.free_blocks;
    r.active_sequence_count = s.active_sequence_count;
    r.active_tokens = s.active_tokens;
    r.resident_tokens = s.resident_tokens;
    r.allocated_token_slots = s.allocated_token_slots;
    r.block_reference_count = s.block_reference_count;
    r.shared_blocks = s.shared_blocks;
    r.sequence_create_count = s.sequence_create_count;
    r.sequence_fork_count = s.sequence_fork_count;
    r.append_count = s.append_count;
    r.release_count = s.release_count;
    r.block_allocation_count = s.block_allocation_count;
    r.block_reuse_count = s.block_reuse_count;
    return r;
  }
  [[nodiscard]] std::size_t bytes_per_token() const noexcept { return impl_->bytes_per_token; }
  [[nodiscard]] std::size_t block_bytes() const noexcept { return impl_->block_bytes; }
  [[nodiscard]] std::size_t token_capacity() const noexcept { return impl_->token_capacity; }
  [[nodiscard]] int device_index() const noexcept { return impl_->device; }
  [[nodiscard]] const PagedKvCacheConfig& config() const noexcept { return impl_->config; }
  /// The C ABI handle (for entry points this header does not wrap).
  [[nodiscard]] helix_paged_cache* native() const noexcept { return impl_->cache; }

 private:
  void check_rows(const Tensor& t, const char* what, std::vector<std::size_t> dims) const {
    detail::require_float_on(t, impl_->device, dims.size(), what);
    for (std::size_t i = 0; i < dims.size(); ++i) {
      if (detail::dim(t, i) != dims[i]) {
        throw_error(ErrorCode::kInvalidArgument, std::string(what) + ": shape mismatch");
      }
    }
  }

  std::shared_ptr<Impl> impl_;
};

using CudaPagedKvCache = HipPagedKvCache;
using CudaPagedSequenceHandle = HipPagedSequenceHandle;

// ------------------------------------------------------------ prefix cache --

/// include/helix/kv_cache/prefix.hpp:15-29.
class PrefixNamespaceId final {
 public:
  PrefixNamespaceId() = default;
  explicit PrefixNamespaceId(std::uint64_t value) noexcept : value_(value) {}
  [[nodiscard]] bool valid() const noexcept { return value_ != 0; }
  [[nodiscard]] std::uint64_t value() const noexcept { return value_; }
  auto operator<=>(const PrefixNamespaceId&) const = default;

 private:
  std::uint64_t value_ = 0;
};

struct PagedPrefixCacheConfig {
  std::size_t maximum_entries = 0;
  std::size_t maximum_block_references = 0;
};

enum class PrefixInsertStatus : std::uint8_t { kInserted, kAlreadyPresent, kRejectedTooLarge };

struct PagedPrefixMatch {
  HipPagedSequenceHandle sequence;  // owned by the caller: release it on the cache
  std::size_t matched_tokens = 0;
};

struct PagedPrefixCacheStats {
  std::size_t maximum_entries = 0, maximum_block_references = 0, entry_count = 0;
  std::size_t retained_tokens = 0, retained_block_references = 0, peak_entries = 0;
  std::size_t peak_block_references = 0;
  std::uint64_t lookup_count = 0, hit_count = 0, miss_count = 0, insertion_count = 0;
  std::uint64_t duplicate_insertion_count = 0, rejected_insertion_count = 0, eviction_count = 0;
  std::uint64_t erase_count = 0;
};

/// include/helix/kv_cache/prefix.hpp:77-113 over the device cache: a bounded
/// index of block-aligned token prefixes to retained anchor sequences; a hit
/// forks the anchor (shared pages, reference counted).  Lock order is prefix
/// cache, then paged cache; do not call while holding a DecodeView of the
/// same cache.
class HipPagedPrefixCache final {
 public:
  HipPagedPrefixCache(std::shared_ptr<HipPagedKvCache> cache, PagedPrefixCacheConfig config)
      : cache_(std::move(cache)) {
    detail::require(cache_ != nullptr, ErrorCode::kInvalidArgument,
                    "HipPagedPrefixCache: cache must not be null");
    const helix_prefix_config c{config.maximum_entries, config.maximum_block_references};
    detail::check(helix_prefix_cache_create(cache_->native(), &c, &prefixes_));
    config_ = config;
    detail::check(helix_prefix_cache_block_tokens(prefixes_, &block_tokens_));
  }
  ~HipPagedPrefixCache() {
    if (prefixes_ != nullptr) helix_prefix_cache_destroy(prefixes_);
  }
  HipPagedPrefixCache(const HipPagedPrefixCache&) = delete;
  HipPagedPrefixCache& operator=(const HipPagedPrefixCache&) = delete;
  HipPagedPrefixCache(HipPagedPrefixCache&&) = delete;
  HipPagedPrefixCache& operator=(HipPagedPrefixCache&&) = delete;

  [[nodiscard]] PrefixInsertStatus insert(PrefixNamespaceId ns, std::span<const std::uint32_t> tokens,
                                          const HipPagedSequenceHandle& source) {
    int status = 0;
    detail::check(helix_prefix_cache_insert(prefixes_, ns.value(), tokens.data(), tokens.size(),
                                            source.native(), &status));
    return static_cast<PrefixInsertStatus>(status);
  }
  [[nodiscard]] std::optional<PagedPrefixMatch> lookup_longest(
      PrefixNamespaceId ns, std::span<const std::uint32_t> tokens,
      std::size_t maximum_prefix_tokens = std::numeric_limits<std::size_t>::max()) {
    int hit = 0;
    helix_sequence s{};
    std::size_t matched = 0;
    detail::check(helix_prefix_cache_lookup_longest(prefixes_, ns.value(), tokens.data(),
                                                    tokens.size(), maximum_prefix_tokens, &hit, &s,
                                                    &matched));
    if (hit == 0) return std::nullopt;
    return PagedPrefixMatch{HipPagedSequenceHandle(s), matched};
  }
  [[nodiscard]] bool contains(PrefixNamespaceId ns, std::span<const std::uint32_t> tokens) const {
    int out = 0;
    detail::check(helix_prefix_cache_contains(prefixes_, ns.value(), tokens.data(), tokens.size(),
                                              &out));
    return out != 0;
  }
  [[nodiscard]] bool erase(PrefixNamespaceId ns, std::span<const std::uint32_t> tokens) {
    int out = 0;
    detail::check(helix_prefix_cache_erase(prefixes_, ns.value(), tokens.data(), tokens.size(),
                                           &out));
    return out != 0;
  }
  [[nodiscard]] bool evict_lru() {
    int out = 0;
    detail::check(helix_prefix_cache_evict_lru(prefixes_, &out));
    return out != 0;
  }
  void clear() { detail::check(helix_prefix_cache_clear(prefixes_)); }
  [[nodiscard]] PagedPrefixCacheStats stats() const {
    helix_prefix_stats s{};
    detail::check(helix_prefix_cache_stats(prefixes_, &s));
    return {s.maximum_entries, s.maximum_block_references, s.entry_count, s.retained_tokens,
            s.retained_block_references, s.peak_entries, s.peak_block_references, s.lookup_count,
            s.hit_count, s.miss_count, s.insertion_count, s.duplicate_insertion_count,
            s.rejected_insertion_count, s.eviction_count, s.erase_count};
  }
  [[nodiscard]] const PagedPrefixCacheConfig& config() const noexcept { return config_; }
  [[nodiscard]] std::size_t block_tokens() const noexcept { return block_tokens_; }

 private:
  std::shared_ptr<HipPagedKvCache> cache_;
  helix_prefix_cache* prefixes_ = nullptr;
  PagedPrefixCacheConfig config_;
  std::size_t block_tokens_ = 0;
};

using PagedPrefixCache = HipPagedPrefixCache;

// ------------------------------------------------------------ decode batch --

/// Extension: the batched decode / chunked-prefill driver of B sequences of
/// one cache (the loop CudaLlamaModel::decode_one_paged_device runs per
/// sequence, src/model/cuda_llama.cpp:365-367, done once for the batch).
/// prepare() reserves each sequence's next slot and uploads the step's
/// tables and lengths; each layer then attends over the pages plus the
/// step's tail rows and, in either order, commits them.  Shapes: query
/// [B, q_heads, D], step keys/values [B, kv_heads, D] (chunk forms take
/// [B, heads, T, D]), all-layer commit [layers, B, kv_heads, D].  The calls
/// of one step share the batch's workspace and step buffers: calls that
/// overlap in time on different streams race, so order them (one stream or
/// events), as a layer loop does.
class DecodeBatch final {
 public:
  DecodeBatch(HipPagedKvCache& cache, std::span<const HipPagedSequenceHandle> sequences,
              std::size_t q_heads, std::size_t max_tokens, std::size_t pages_per_split = 0)
      : device_(cache.device_index()),
        batch_(sequences.size()),
        q_heads_(q_heads),
        kv_heads_(cache.config().kv_heads),
        head_dim_(cache.config().head_dimension),
        layers_(cache.config().layers) {
    std::vector<helix_sequence> raw(sequences.size());
    for (std::size_t i = 0; i < raw.size(); ++i) raw[i] = sequences[i].native();
    detail::check(helix_decode_batch_create(cache.native(), raw.data(), raw.size(), q_heads,
                                            max_tokens, pages_per_split, &batch_handle_));
  }
  ~DecodeBatch() {
    if (batch_handle_ != nullptr) helix_decode_batch_destroy(batch_handle_);
  }
  DecodeBatch(const DecodeBatch&) = delete;
  DecodeBatch& operator=(const DecodeBatch&) = delete;

  /// A one-token step: append_layer() then takes [B, kv_heads, D] rows and
  /// prefill_layer() [B, heads, 1, D] rows.
  void prepare(const hip::Stream& stream) {
    step_tokens_ = 0;  // a failed prepare leaves the batch unprepared
    detail::check(helix_decode_batch_prepare(batch_handle_, stream.native()));
    step_tokens_ = 1;
    chunked_ = false;
  }
  void prepare_chunk(std::size_t tokens, const hip::Stream& stream) {
    step_tokens_ = 0;
    detail::check(helix_decode_batch_prepare_chunk(batch_handle_, tokens, stream.native()));
    step_tokens_ = tokens;
    chunked_ = true;
  }
  void rope(Tensor& query, Tensor& key, const Tensor& cosine, const Tensor& sine,
            const hip::Stream& stream) {
    rows(query, "rope query", q_heads_);
    rows(key, "rope key", kv_heads_);
    detail::require_float_on(cosine, device_, 2, "rope cosine");
    detail::require_float_on(sine, device_, 2, "rope sine");
    detail::require(cosine.shape() == sine.shape() && detail::dim(cosine, 1) * 2 == head_dim_,
                    ErrorCode::kInvalidArgument, "rope: tables must be [rows, head_dim / 2]");
    detail::check(helix_decode_batch_rope(batch_handle_, query.data<float>(), key.data<float>(),
                                          cosine.data_as<float>(), sine.data_as<float>(),
                                          detail::dim(cosine, 0), stream.native()));
  }
  void attention_layer(std::size_t layer, const Tensor& query, const Tensor& tail_key,
                       const Tensor& tail_value, Tensor& output, const hip::Stream& stream) {
    rows(query, "query", q_heads_);
    rows(tail_key, "tail key", kv_heads_);
    rows(tail_value, "tail value", kv_heads_);
    rows(output, "output", q_heads_);
    detail::check(helix_decode_batch_attention_layer(
        batch_handle_, layer, query.data_as<float>(), tail_key.data_as<float>(),
        tail_value.data_as<float>(), output.data<float>(), stream.native()));
  }
  void append_attention_layer(std::size_t layer, const Tensor& query, const Tensor& keys,
                              const Tensor& values, Tensor& output, const hip::Stream& stream) {
    rows(query, "query", q_heads_);
    rows(keys, "keys", kv_heads_);
    rows(values, "values", kv_heads_);
    rows(output, "output", q_heads_);
    detail::check(helix_decode_batch_append_attention_layer(
        batch_handle_, layer, query.data_as<float>(), keys.data_as<float>(),
        values.data_as<float>(), output.data<float>(), stream.native()));
  }
  /// The step's rows of one layer: [B, kv_heads, D] after prepare(),
  /// [B, kv_heads, T, D] after prepare_chunk(T).
  void append_layer(std::size_t layer, const Tensor& keys, const Tensor& values,
                    const hip::Stream& stream) {
    if (!chunked_) {
      rows(keys, "keys", kv_heads_);
      rows(values, "values", kv_heads_);
    } else {
      chunk_rows(keys, "chunk keys", kv_heads_);
      chunk_rows(values, "chunk values", kv_heads_);
    }
    detail::check(helix_decode_batch_append_layer(batch_handle_, layer, keys.data_as<float>(),
                                                  values.data_as<float>(), stream.native()));
  }
  /// Every layer's rows: [layers, B, kv_heads, D] after prepare(),
  /// [layers, B, kv_heads, T, D] after prepare_chunk(T).
  void append_all_layers(const Tensor& keys, const Tensor& values, const hip::Stream& stream) {
    for (const Tensor* t : {&keys, &values}) {
      const std::size_t rank = chunked_ ? 5 : 4;
      detail::require_float_on(*t, device_, rank, "append_all_layers");
      detail::require(detail::dim(*t, 0) == layers_ && detail::dim(*t, 1) == batch_ &&
                          detail::dim(*t, 2) == kv_heads_ &&
                          (!chunked_ || detail::dim(*t, 3) == step_tokens_) &&
                          detail::dim(*t, rank - 1) == head_dim_,
                      ErrorCode::kInvalidArgument,
                      "append_all_layers: rows must be [layers, batch, kv_heads, (tokens,) head_dim]");
    }
    detail::check(helix_decode_batch_append_all_layers(batch_handle_, keys.data_as<float>(),
                                                       values.data_as<float>(), stream.native()));
  }
  void prefill_layer(std::size_t layer, const Tensor& query, const Tensor& chunk_key,
                     const Tensor& chunk_value, Tensor& output, const hip::Stream& stream) {
    chunk_rows(query, "prefill query", q_heads_);
    chunk_rows(chunk_key, "prefill key", kv_heads_);
    chunk_rows(chunk_value, "prefill value", kv_heads_);
    chunk_rows(output, "prefill output", q_heads_);
    detail::check(helix_decode_batch_prefill_layer(
        batch_handle_, layer, query.data_as<float>(), chunk_key.data_as<float>(),
        chunk_value.data_as<float>(), output.data<float>(), stream.native()));
  }
  [[nodiscard]] std::size_t shared_pages() const {
    std::size_t n = 0;
    detail::check(helix_decode_batch_shared_pages(batch_handle_, &n));
    return n;
  }
  [[nodiscard]] std::size_t batch() const noexcept { return batch_; }

 private:
  void rows(const Tensor& t, const char* what, std::size_t heads) const {
    detail::require_float_on(t, device_, 3, what);
    detail::require(detail::dim(t, 0) == batch_ && detail::dim(t, 1) == heads &&
                        detail::dim(t, 2) == head_dim_,
                    ErrorCode::kInvalidArgument, "DecodeBatch: rows must be [batch, heads, head_dim]");
  }
  void chunk_rows(const Tensor& t, const char* what, std::size_t heads) const {
    detail::require(step_tokens_ != 0, ErrorCode::kInvalidArgument,
                    "DecodeBatch: prepare() or prepare_chunk() must precede the step's calls");
    detail::require_float_on(t, device_, 4, what);
    detail::require(detail::dim(t, 0) == batch_ && detail::dim(t, 1) == heads &&
                        detail::dim(t, 2) == step_tokens_ && detail::dim(t, 3) == head_dim_,
                    ErrorCode::kInvalidArgument,
                    "DecodeBatch: chunk rows must be [batch, heads, tokens, head_dim]");
  }

  helix_decode_batch* batch_handle_ = nullptr;
  int device_;
  std::size_t batch_, q_heads_, kv_heads_, head_dim_, layers_;
  std::size_t step_tokens_ = 0;  // tokens of the prepared step, 0: not prepared
  bool chunked_ = false;         // prepared by prepare_chunk()
};

}  // namespace kv_cache

// --------------------------------------------------------------- attention --

namespace attention::hip {

using PagedBlockTable = kv_cache::hip::PagedBlockTable;
using Stream = helix_amd::hip::Stream;

namespace detail {

using helix_amd::detail::dim;

/// Rank, dtype and device of the reference's operands: query [H, T, Dk],
/// key blocks [N, Hkv, P, Dk], value blocks [N, Hkv, P, Dv], a valid table
/// whose capacity is N (src/attention/cuda_paged.cu:211-352).
inline int check_operands(const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
                          const PagedBlockTable& table) {
  const int device = key_blocks.device().index;
  helix_amd::detail::require_float_on(query, device, 3, "paged attention query");
  helix_amd::detail::require_float_on(key_blocks, device, 4, "paged attention key blocks");
  helix_amd::detail::require_float_on(value_blocks, device, 4, "paged attention value blocks");
  helix_amd::detail::require(table.valid(), ErrorCode::kInvalidArgument,
                             "paged attention: block table is not valid (moved from)");
  helix_amd::detail::require(table.device_index() == device, ErrorCode::kInvalidArgument,
                             "paged attention: block table is on another device");
  helix_amd::detail::require(
      dim(key_blocks, 3) == dim(query, 2), ErrorCode::kInvalidArgument,
      "paged attention: key blocks width must equal the query width");
  for (std::size_t i = 0; i < 3; ++i) {
    helix_amd::detail::require(dim(value_blocks, i) == dim(key_blocks, i),
                               ErrorCode::kInvalidArgument,
                               "paged attention: value blocks must match key blocks [N, H, P]");
  }
  helix_amd::detail::require(table.physical_block_count() == dim(key_blocks, 0),
                             ErrorCode::kInvalidArgument,
                             "paged attention: block table capacity must equal the pool's blocks");
  return device;
}

inline void check_tail(const Tensor& query, const Tensor& value_blocks, const Tensor& tail_key,
                       const Tensor& tail_value, int device) {
  helix_amd::detail::require_float_on(tail_key, device, 3, "paged attention tail key");
  helix_amd::detail::require_float_on(tail_value, device, 3, "paged attention tail value");
  // [kv_heads, T, D]: with as many query as kv heads (the reference's only
  // case) the query's own shape; grouped-query attention is an extension.
  helix_amd::detail::require(
      dim(tail_key, 0) == dim(value_blocks, 1) && dim(tail_key, 1) == dim(query, 1) &&
          dim(tail_key, 2) == dim(query, 2),
      ErrorCode::kInvalidArgument, "paged attention: tail key must be [Hkv, T, Dk]");
  helix_amd::detail::require(
      dim(tail_value, 0) == dim(value_blocks, 1) && dim(tail_value, 1) == dim(query, 1) &&
          dim(tail_value, 2) == dim(value_blocks, 3),
      ErrorCode::kInvalidArgument, "paged attention: tail value must be [Hkv, T, Dv]");
}

inline Shape output_shape(const Tensor& query, const Tensor& value_blocks) {
  return {query.shape()[0], query.shape()[1], value_blocks.shape()[3]};
}

inline void check_output(const Tensor& output, const Shape& shape, int device, const char* what) {
  helix_amd::detail::require_float_on(output, device, 3, what);
  helix_amd::detail::require(output.shape() == shape, ErrorCode::kInvalidArgument,
                             "paged attention: output/workspace shape mismatch");
}

}  // namespace detail

/// include/helix/attention/cuda_paged.hpp:15-22: [H, T, kv_tokens].
[[nodiscard]] inline Shape paged_score_workspace_shape(const Tensor& query, const Tensor& key_blocks,
                                                       const PagedBlockTable& block_table,
                                                       std::size_t kv_tokens) {
  detail::check_operands(query, key_blocks, key_blocks, block_table);
  std::size_t bytes = 0;
  helix_amd::detail::check(helix_paged_score_workspace_bytes(
      detail::dim(query, 0), detail::dim(query, 1), detail::dim(key_blocks, 1),
      detail::dim(key_blocks, 0), detail::dim(key_blocks, 2), block_table.logical_block_count(),
      kv_tokens, &bytes));
  return {query.shape()[0], query.shape()[1], static_cast<Dimension>(kv_tokens)};
}

[[nodiscard]] inline std::size_t paged_score_workspace_bytes(const Tensor& query,
                                                             const Tensor& key_blocks,
                                                             const PagedBlockTable& block_table,
                                                             std::size_t kv_tokens) {
  return shape_numel(paged_score_workspace_shape(query, key_blocks, block_table, kv_tokens)) *
         sizeof(float);
}

/// include/helix/attention/cuda_paged.hpp:24-38: [H, T, history + T].
[[nodiscard]] inline Shape paged_tail_score_workspace_shape(
    const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
    const PagedBlockTable& block_table, std::size_t history_tokens, const Tensor& tail_key,
    const Tensor& tail_value) {
  const int device = detail::check_operands(query, key_blocks, value_blocks, block_table);
  detail::check_tail(query, value_blocks, tail_key, tail_value, device);
  std::size_t bytes = 0;
  helix_amd::detail::check(helix_paged_tail_score_workspace_bytes(
      detail::dim(query, 0), detail::dim(query, 1), detail::dim(key_blocks, 1),
      detail::dim(key_blocks, 0), detail::dim(key_blocks, 2), block_table.logical_block_count(),
      history_tokens, &bytes));
  return {query.shape()[0], query.shape()[1],
          static_cast<Dimension>(history_tokens + detail::dim(query, 1))};
}

[[nodiscard]] inline std::size_t paged_tail_score_workspace_bytes(
    const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
    const PagedBlockTable& block_table, std::size_t history_tokens, const Tensor& tail_key,
    const Tensor& tail_value) {
  return shape_numel(paged_tail_score_workspace_shape(query, key_blocks, value_blocks, block_table,
                                                      history_tokens, tail_key, tail_value)) *
         sizeof(float);
}

/// include/helix/attention/cuda_paged.hpp:40-47: causal attention of T
/// queries at positions offset.. over kv_tokens paged tokens; the workspace
/// receives the probabilities.
inline void paged_scaled_dot_product_attention_out(
    const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
    const PagedBlockTable& block_table, std::size_t kv_tokens, std::size_t query_position_offset,
    Tensor& output, Tensor& score_workspace, const Stream& stream) {
  const int device = detail::check_operands(query, key_blocks, value_blocks, block_table);
  detail::check_output(output, detail::output_shape(query, value_blocks), device,
                       "paged attention output");
  helix_amd::detail::require_float_on(score_workspace, device, 3, "paged attention workspace");
  helix_amd::detail::check(helix_paged_attention_out(
      query.data_as<float>(), detail::dim(query, 0), detail::dim(query, 1), detail::dim(query, 2),
      key_blocks.data_as<float>(), value_blocks.data_as<float>(), detail::dim(key_blocks, 0),
      detail::dim(key_blocks, 1), detail::dim(key_blocks, 2), detail::dim(value_blocks, 3),
      block_table.data(), block_table.logical_block_count(), kv_tokens, query_position_offset,
      output.data<float>(), score_workspace.data<float>(), score_workspace.numel(),
      stream.native()));
}

namespace detail {
using TailEntry = int (*)(const float*, size_t, size_t, size_t, const float*, const float*,
                          size_t, size_t, size_t, size_t, const uint32_t*, size_t, size_t,
                          const float*, const float*, float*, float*, size_t, helix_stream);
inline void with_tail_out(TailEntry entry, const Tensor& query, const Tensor& key_blocks,
                          const Tensor& value_blocks, const PagedBlockTable& block_table,
                          std::size_t history_tokens, const Tensor& tail_key,
                          const Tensor& tail_value, Tensor& output, Tensor& score_workspace,
                          const Stream& stream) {
  const int device = check_operands(query, key_blocks, value_blocks, block_table);
  check_tail(query, value_blocks, tail_key, tail_value, device);
  check_output(output, output_shape(query, value_blocks), device, "paged attention output");
  helix_amd::detail::require_float_on(score_workspace, device, 3, "paged attention workspace");
  helix_amd::detail::check(entry(
      query.data_as<float>(), detail::dim(query, 0), detail::dim(query, 1), detail::dim(query, 2),
      key_blocks.data_as<float>(), value_blocks.data_as<float>(), detail::dim(key_blocks, 0),
      detail::dim(key_blocks, 1), detail::dim(key_blocks, 2), detail::dim(value_blocks, 3),
      block_table.data(), block_table.logical_block_count(), history_tokens,
      tail_key.data_as<float>(), tail_value.data_as<float>(), output.data<float>(),
      score_workspace.data<float>(), score_workspace.numel(), stream.native()));
}
}  // namespace detail

/// include/helix/attention/cuda_paged.hpp:49-60: T tail queries at
/// positions history.. attend over the history pages and, causally, the
/// uncommitted tail rows; the workspace receives the probabilities.  At
/// head_dim 128 with 16-token pages a one-token decode runs the single-sequence
/// decode kernel and a chunk the matrix-core prefill kernel.
inline void paged_scaled_dot_product_attention_with_tail_out(
    const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
    const PagedBlockTable& block_table, std::size_t history_tokens, const Tensor& tail_key,
    const Tensor& tail_value, Tensor& output, Tensor& score_workspace, const Stream& stream) {
  detail::with_tail_out(&helix_paged_attention_with_tail_out, query, key_blocks, value_blocks,
                        block_table, history_tokens, tail_key, tail_value, output,
                        score_workspace, stream);
}

/// The same call on the exact scalar kernel for every shape (the
/// reference's loop order, no device scratch); the workspace [heads, tail,
/// history + tail] receives the probabilities.
inline void paged_scaled_dot_product_attention_with_tail_probabilities_out(
    const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
    const PagedBlockTable& block_table, std::size_t history_tokens, const Tensor& tail_key,
    const Tensor& tail_value, Tensor& output, Tensor& score_workspace, const Stream& stream) {
  detail::with_tail_out(&helix_paged_attention_with_tail_probabilities_out, query, key_blocks,
                        value_blocks, block_table, history_tokens, tail_key, tail_value, output,
                        score_workspace, stream);
}

/// include/helix/attention/cuda_paged.hpp:62-69: allocating form; returns
/// after the stream has finished.
[[nodiscard]] inline Tensor paged_scaled_dot_product_attention(
    const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
    const PagedBlockTable& block_table, std::size_t kv_tokens, std::size_t query_position_offset,
    const Stream& stream) {
  const Shape ws = paged_score_workspace_shape(query, key_blocks, block_table, kv_tokens);
  const Device device = key_blocks.device();
  Tensor output = Tensor::empty(detail::output_shape(query, value_blocks), DType::kFloat32, device);
  Tensor workspace = Tensor::empty(ws, DType::kFloat32, device);
  paged_scaled_dot_product_attention_out(query, key_blocks, value_blocks, block_table, kv_tokens,
                                         query_position_offset, output, workspace, stream);
  stream.synchronize();
  return output;
}

/// include/helix/attention/cuda_paged.hpp:71-76: allocating form.
[[nodiscard]] inline Tensor paged_scaled_dot_product_attention_with_tail(
    const Tensor& query, const Tensor& key_blocks, const Tensor& value_blocks,
    const PagedBlockTable& block_table, std::size_t history_tokens, const Tensor& tail_key,
    const Tensor& tail_value, const Stream& stream) {
  const Shape ws = paged_tail_score_workspace_shape(query, key_blocks, value_blocks, block_table,
                                                    history_tokens, tail_key, tail_value);
  const Device device = key_blocks.device();
  Tensor output = Tensor::empty(detail::output_shape(query, value_blocks), DType::kFloat32, device);
  Tensor workspace = Tensor::empty(ws, DType::kFloat32, device);
  paged_scaled_dot_product_attention_with_tail_out(query, key_blocks, value_blocks, block_table,
                                                   history_tokens, tail_key, tail_value, output,
                                                   workspace, stream);
  stream.synchronize();
  return output;
}

}  // namespace attention::hip
namespace attention {
namespace cuda = hip;
}

}  // namespace helix_amd

#endif /* HELIX_PAGED_HPP */
