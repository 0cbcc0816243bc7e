// Implementation of the restated runtime contract (kidi_runtime.hpp): tensor storage on the host or a HIP device,
// operation names, the output pool and the defaults of Operator / OperatorBackend (runtime/operator.cpp:10-76).
#include "kidi_runtime.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace kidi::tensor {

auto element_size(DType dtype) noexcept -> std::size_t {
    switch (dtype) {
        case DType::BOOL: case DType::U8: case DType::I8: case DType::E4M3: case DType::E5M2: return 1;
        case DType::U16: case DType::I16: case DType::F16: case DType::BF16: return 2;
        case DType::U32: case DType::I32: case DType::F32: return 4;
        case DType::U64: case DType::I64: case DType::F64: return 8;
    }
    return 0;
}

Tensor::Storage::~Storage() {
    if (!owned || !data) return;
    if (kind == DeviceKind::HIP) (void)hipFree(data);
    else std::free(data);
}

auto Tensor::element_count() const noexcept -> std::int64_t {
    std::int64_t n = 1;
    for (const auto d : shape_) n *= d;
    return n;
}

auto Tensor::empty(std::vector<std::int64_t> shape, DType dtype, Device device) -> Tensor {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.device_ = device;
    t.storage_ = std::make_shared<Storage>();
    t.storage_->owned = true;
    t.storage_->kind = device.kind;
    const std::size_t bytes = std::max<std::size_t>(t.nbytes(), 1);
    if (device.kind == DeviceKind::HIP) {
        int prev = 0;
        (void)hipGetDevice(&prev);
        (void)hipSetDevice(device.index);
        const hipError_t e = hipMalloc(&t.storage_->data, bytes);
        (void)hipSetDevice(prev);
        if (e != hipSuccess) ops::fail(core::ErrorCode::RUNTIME, std::string("hipMalloc failed: ") + hipGetErrorString(e));
    } else if (device.kind == DeviceKind::CPU) {
        t.storage_->data = std::aligned_alloc(64, (bytes + 63) / 64 * 64);
        if (!t.storage_->data) ops::fail(core::ErrorCode::RUNTIME, "host allocation failed");
    } else {
        ops::fail(core::ErrorCode::UNSUPPORTED, "tensor storage on this device kind is not available");
    }
    return t;
}

auto Tensor::borrow(void* data, std::vector<std::int64_t> shape, DType dtype, Device device) -> Tensor {
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.device_ = device;
    t.storage_ = std::make_shared<Storage>();
    t.storage_->data = data;
    t.storage_->kind = device.kind;
    return t;
}

}  // namespace kidi::tensor

namespace kidi::runtime {

auto operation_name(Operation operation) -> std::string_view {
    static constexpr std::array<std::string_view, 39> names{
        "add", "multiply", "cast", "matmul", "linear", "quantized_linear", "gelu", "layer_norm", "softmax",
        "log_softmax", "transpose", "slice", "gather", "concat", "scatter", "attention", "residual_norm", "rms_norm",
        "tanh", "rotary", "packed_linear", "rms_norm_residual", "static_round", "greedy_token", "rms_rotary",
        "gelu_multiply", "silu_multiply", "silu_gate", "embedding", "gated_feed_forward", "diffusion_candidates",
        "diffusion_update", "embedding_sum", "conv1d", "snake_conv1d", "snake_quantized_linear", "conv_transpose_fold",
        "snake", "gelu_gate"};
    const auto i = static_cast<std::size_t>(operation);
    if (i >= names.size()) throw std::out_of_range("operation");
    return names[i];
}

auto Operator::run_into(TensorInputs, std::span<tensor::Tensor>) -> void {
    ops::fail(core::ErrorCode::UNSUPPORTED, "this backend cannot replay captured steps");
}

auto copy_tensor(tensor::Tensor& destination, const tensor::Tensor& source) -> void {
    if (destination.nbytes() != source.nbytes() || destination.dtype() != source.dtype())
        ops::fail(core::ErrorCode::INVALID_ARGUMENT, "tensor copy shape or dtype mismatch");
    const bool dst_dev = destination.device().kind == tensor::DeviceKind::HIP;
    const bool src_dev = source.device().kind == tensor::DeviceKind::HIP;
    const hipMemcpyKind kind = dst_dev ? (src_dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice)
                                       : (src_dev ? hipMemcpyDeviceToHost : hipMemcpyHostToHost);
    if (const hipError_t e = hipMemcpy(destination.data(), source.data(), source.nbytes(), kind); e != hipSuccess)
        ops::fail(core::ErrorCode::RUNTIME, std::string("hipMemcpy failed: ") + hipGetErrorString(e));
}

auto OperatorBackend::stage_inputs(std::span<const tensor::Tensor> inputs, tensor::Device device)
    -> std::vector<tensor::Tensor> {
    std::vector<tensor::Tensor> staged;
    staged.reserve(inputs.size());
    for (const auto& input : inputs) {
        if (input.device() == device) {
            staged.push_back(input);
            continue;
        }
        auto copy = tensor::Tensor::empty(input.shape_vector(), input.dtype(), device);
        copy_tensor(copy, input);
        staged.push_back(copy);
    }
    return staged;
}

auto OutputPool::acquire(std::span<const std::int64_t> shape, tensor::DType dtype, tensor::Device device)
    -> tensor::Tensor {
    for (const auto& buffer : buffers_)
        if (buffer.owns_unique_storage() && buffer.dtype() == dtype && buffer.device() == device &&
            std::ranges::equal(buffer.shape(), shape))
            return buffer;
    auto output = tensor::Tensor::empty({shape.begin(), shape.end()}, dtype, device);
    ++allocations_.count;
    allocations_.bytes += output.nbytes();
    buffers_.push_back(output);
    return output;
}

}  // namespace kidi::runtime
