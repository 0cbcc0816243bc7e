// C++20 restatement of the parts of Kidi's runtime contract that a PACKED_LINEAR plug-in touches, so the HIP
// adapter (packed_linear.cpp) compiles and is tested here exactly as a Kidi maintainer would write it:
//   core::ErrorCode / core::Error           src/kidi/core/error.h:8-19
//   ops::Failure                            src/kidi/ops/context.h:52-59
//   tensor::DType, tensor::DeviceKind       src/kidi/tensor/dtype.h:10-26, tensor/device.h:14-22
//   runtime::TensorInputs .. OutputPool     src/kidi/runtime/operator.h:17-153, runtime/operator.cpp:10-76
//   graph::Compiler::prepare_operator       src/kidi/graph/compiler.h:37-40
// Names, argument meaning and error behaviour follow the reference. tensor::Tensor is a minimal stand-in for Kidi's
// (shape, dtype, device, shared storage on the host or on a HIP device); DeviceKind gains HIP, the device kind a
// maintainer adds for this backend.
#pragma once

#include <array>
#include <cstdint>
#include <initializer_list>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace kidi::core {
enum class ErrorCode { INVALID_ARGUMENT, IO, INVALID_MANIFEST, UNSUPPORTED, RUNTIME };
struct Error {
    ErrorCode code;
    std::string message;
};
}  // namespace kidi::core

namespace kidi::ops {
class Failure : public std::runtime_error {
public:
    explicit Failure(core::Error error) : std::runtime_error(error.message), error_(std::move(error)) {}
    auto error() const noexcept -> const core::Error& { return error_; }

private:
    core::Error error_;
};
[[noreturn]] inline void fail(core::ErrorCode code, std::string message) { throw Failure({code, std::move(message)}); }
}  // namespace kidi::ops

namespace kidi::tensor {
enum class DType { BOOL, U8, I8, U16, I16, U32, I32, U64, I64, F16, BF16, F32, F64, E4M3, E5M2 };
auto element_size(DType dtype) noexcept -> std::size_t;

enum class DeviceKind { CPU, Q_NPU, CUDA, A_GPU, WEB_GPU, VULKAN, HIP, COUNT };
struct Device {
    DeviceKind kind = DeviceKind::CPU;
    int index = 0;
    auto operator==(const Device&) const -> bool = default;
};

// Shared storage (host memory, or HIP device memory) behind a shape and a dtype. Copies share the storage.
class Tensor {
public:
    Tensor() = default;
    static auto empty(std::vector<std::int64_t> shape, DType dtype, Device device) -> Tensor;
    // a view of memory the caller owns (no ownership taken)
    static auto borrow(void* data, std::vector<std::int64_t> shape, DType dtype, Device device) -> Tensor;

    auto defined() const noexcept -> bool { return static_cast<bool>(storage_); }
    auto data() const noexcept -> void* { return storage_ ? storage_->data : nullptr; }
    auto shape() const noexcept -> std::span<const std::int64_t> { return shape_; }
    auto shape_vector() const -> std::vector<std::int64_t> { return shape_; }
    auto dimensions() const noexcept -> std::size_t { return shape_.size(); }
    auto size(std::int64_t dim) const -> std::int64_t { return shape_.at(dim < 0 ? shape_.size() + dim : dim); }
    auto element_count() const noexcept -> std::int64_t;
    auto nbytes() const noexcept -> std::size_t { return static_cast<std::size_t>(element_count()) * element_size(dtype_); }
    auto dtype() const noexcept -> DType { return dtype_; }
    auto device() const noexcept -> Device { return device_; }
    // true when no other Tensor shares this storage (OutputPool hands such buffers out again)
    auto owns_unique_storage() const noexcept -> bool { return storage_ && storage_.use_count() == 1; }

private:
    struct Storage {
        void* data = nullptr;
        bool owned = false;
        DeviceKind kind = DeviceKind::CPU;
        ~Storage();
    };
    std::shared_ptr<Storage> storage_;
    std::vector<std::int64_t> shape_;
    DType dtype_ = DType::F32;
    Device device_{};
};
}  // namespace kidi::tensor

namespace kidi::graph {
class Compiler;
}

namespace kidi::runtime {
/// Borrowed operands, either a contiguous tensor span or a list of tensor addresses (operator.h:18-42).
class TensorInputs {
public:
    TensorInputs(std::span<const tensor::Tensor> inputs) : contiguous_(inputs.data()), size_(inputs.size()) {}
    TensorInputs(std::initializer_list<const tensor::Tensor*> inputs) : indirect_(inputs), size_(inputs.size()) {}
    TensorInputs(const std::vector<tensor::Tensor>& inputs) : TensorInputs(std::span<const tensor::Tensor>(inputs)) {}
    auto operator[](std::size_t index) const -> const tensor::Tensor& {
        return indirect_.size() != 0 ? *indirect_.begin()[index] : contiguous_[index];
    }
    auto front() const -> const tensor::Tensor& { return (*this)[0]; }
    auto back() const -> const tensor::Tensor& { return (*this)[size_ - 1]; }
    auto size() const noexcept -> std::size_t { return size_; }
    auto first(std::size_t count) const -> TensorInputs {
        auto result = *this;
        result.size_ = count;
        return result;
    }

private:
    const tensor::Tensor* contiguous_ = nullptr;
    std::initializer_list<const tensor::Tensor*> indirect_;
    std::size_t size_;
};

enum class Operation {
    ADD, MULTIPLY, CAST, MATMUL, LINEAR, QUANTIZED_LINEAR, GELU, LAYER_NORM, SOFTMAX, LOG_SOFTMAX, TRANSPOSE, SLICE,
    GATHER, CONCAT, SCATTER, ATTENTION, RESIDUAL_NORM, RMS_NORM, TANH, ROTARY, PACKED_LINEAR, RMS_NORM_RESIDUAL,
    STATIC_ROUND, GREEDY_TOKEN, RMS_ROTARY, GELU_MULTIPLY, SILU_MULTIPLY, SILU_GATE, EMBEDDING, GATED_FEED_FORWARD,
    DIFFUSION_CANDIDATES, DIFFUSION_UPDATE, EMBEDDING_SUM, CONV1D, SNAKE_CONV1D, SNAKE_QUANTIZED_LINEAR,
    CONV_TRANSPOSE_FOLD, SNAKE, GELU_GATE
};
auto operation_name(Operation operation) -> std::string_view;

struct BlockwiseQuantizationSpec {
    std::span<const float> scales;
    std::span<const std::int32_t> zero_points;
    std::size_t block_size = 0;
};
struct OperatorSpec {
    Operation operation;
    std::span<const std::int64_t> attributes;
    tensor::DType dtype = tensor::DType::F32;
    float epsilon = 0;
    bool dynamic_parameters = false;
    bool packed_prefill = false;
    bool vector_projection = false;
    std::array<BlockwiseQuantizationSpec, 2> quantization;
};

struct AllocationStats {
    std::uint64_t count = 0;
    std::uint64_t bytes = 0;
};

class Operator {
public:
    virtual ~Operator() = default;
    virtual auto run(TensorInputs inputs) -> tensor::Tensor = 0;
    virtual auto run_(TensorInputs inputs, tensor::Tensor& destination) -> tensor::Tensor = 0;
    virtual auto run_pair(TensorInputs inputs) -> std::array<tensor::Tensor, 2> { return {tensor::Tensor{}, run(inputs)}; }
    /// Writes into caller-owned outputs with the prepared shapes; UNSUPPORTED unless an operator overrides it.
    virtual auto run_into(TensorInputs inputs, std::span<tensor::Tensor> outputs) -> void;
    virtual auto allocations() const -> AllocationStats { return {}; }
    virtual auto release_workspaces() -> void {}
};

class OperatorBackend {
public:
    virtual ~OperatorBackend() = default;
    virtual auto prepare(const OperatorSpec&, TensorInputs) -> std::unique_ptr<Operator> = 0;
    virtual auto synchronize() -> void = 0;
    virtual auto release_cached_buffers() -> void {}
    virtual auto activation_dtype(tensor::DType) const noexcept -> tensor::DType { return tensor::DType::F32; }
    /// True when every prepared operator implements `run_into`, so captured steps can replay.
    virtual auto supports_replay() const noexcept -> bool { return false; }
    virtual auto graph_compiler() -> std::shared_ptr<graph::Compiler> { return {}; }
    virtual auto stage_inputs(std::span<const tensor::Tensor> inputs, tensor::Device device) -> std::vector<tensor::Tensor>;
    virtual auto copy_slice_(tensor::Tensor& destination, const tensor::Tensor& source, std::size_t outer,
                             std::size_t source_bytes, std::size_t destination_bytes, std::size_t offset_bytes) -> void = 0;
};

/// Output buffers an operator hands out again once nothing else holds them (operator.cpp:64-76).
class OutputPool {
public:
    OutputPool() { buffers_.reserve(32); }
    auto acquire(std::span<const std::int64_t> shape, tensor::DType dtype, tensor::Device device) -> tensor::Tensor;
    auto allocations() const -> AllocationStats { return allocations_; }
    auto clear() -> void { buffers_.clear(); }

private:
    std::vector<tensor::Tensor> buffers_;
    AllocationStats allocations_;
};

// host <-> device copy of a whole tensor (same shape and dtype)
auto copy_tensor(tensor::Tensor& destination, const tensor::Tensor& source) -> void;
}  // namespace kidi::runtime

namespace kidi::graph {
/// The interceptor hook Context::Impl::run consults before the backend (compiler.h:37-40; context.cpp:366): a
/// non-null operator replaces the backend's for this spec.
class Compiler {
public:
    virtual ~Compiler() = default;
    virtual auto name() const -> std::string_view = 0;
    virtual auto supports_step_operation(runtime::Operation) const -> bool { return true; }
    virtual auto prepare_operator(const runtime::OperatorSpec&, runtime::TensorInputs) -> std::unique_ptr<runtime::Operator> {
        return nullptr;
    }
};
}  // namespace kidi::graph
