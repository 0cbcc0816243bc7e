// The PACKED_LINEAR plug-in a Kidi maintainer adds for MI355X, compiled against the restated contract
// (kidi_runtime.hpp) and the C ABI (include/kq.h):
//   hip::PackedLinear  runtime::Operator for Operation::PACKED_LINEAR (ops/context.cpp:932-937 builds its spec:
//                      attributes {bits, group_size, bit_cast<int32>(output_scale)}, dtype F32, epsilon =
//                      input_scale, inputs {input, weight, scales[, bound zero]}); the weight is packed once at
//                      prepare (kq_weight_pack), run / run_into call kq_packed_linear, run_ is UNSUPPORTED
//   hip::Compiler      graph::Compiler interceptor that claims PACKED_LINEAR and declines everything else, the
//                      hook Context::Impl::run consults before the backend (ops/context.cpp:366)
//   hip::HipOperators  runtime::OperatorBackend whose prepare builds PackedLinear (other operations UNSUPPORTED)
// Device tensors run stream-ordered on the backend's stream; host tensors (a CPU-device graph) are staged to the GPU
// and the result is copied back before run returns, as Kidi's CPU device expects.
// The extern "C" kqa_* functions at the end exist for tests: they drive the adapter through raw pointers (status =
// core::ErrorCode + 1, as kq_status).
#include <hip/hip_runtime.h>

#include <bit>
#include <cstring>
#include <string>

#include "../../include/kq.h"
#include "kidi_runtime.hpp"

namespace kidi::runtime::hip {

using core::ErrorCode;
using tensor::DeviceKind;
using tensor::DType;
using tensor::Tensor;

[[noreturn]] void raise(kq_status s) { ops::fail(static_cast<ErrorCode>(s - 1), kq_last_error()); }

kq_dtype kq_dtype_of(DType dtype) {
    switch (dtype) {
        case DType::F32: return KQ_F32;
        case DType::F16: return KQ_F16;
        case DType::BF16: return KQ_BF16;
        case DType::U8: return KQ_U8;
        case DType::I8: return KQ_I8;
        default: return KQ_NONE;
    }
}

class PackedLinear final : public Operator {
public:
    PackedLinear(const OperatorSpec& spec, TensorInputs in, hipStream_t stream, tensor::Device)
        : stream_(stream) {
        // the weight and every staging buffer live on the current HIP device, whatever the graph's device is
        int hip_device = 0;
        if (const hipError_t e = hipGetDevice(&hip_device); e != hipSuccess)
            ops::fail(ErrorCode::RUNTIME, std::string("hipGetDevice failed: ") + hipGetErrorString(e));
        device_ = {DeviceKind::HIP, hip_device};
        if (spec.operation != Operation::PACKED_LINEAR || spec.attributes.size() < 3 || (in.size() != 3 && in.size() != 4))
            ops::fail(ErrorCode::INVALID_ARGUMENT, "packed linear shape or dtype mismatch");
        const Tensor& x = in[0];
        const Tensor& W = in[1];
        const Tensor& S = in[2];
        if (x.dimensions() == 0 || W.dimensions() != 2 || S.dimensions() != 2)
            ops::fail(ErrorCode::INVALID_ARGUMENT, "packed linear shape or dtype mismatch");
        const bool on_device = W.device().kind == DeviceKind::HIP;
        if ((S.device().kind == DeviceKind::HIP) != on_device || (in.size() == 4 && (in[3].device().kind == DeviceKind::HIP) != on_device))
            ops::fail(ErrorCode::INVALID_ARGUMENT, "packed weight parts must share one device");
        kq_pack_desc d{};
        d.bits = static_cast<std::int32_t>(spec.attributes[0]);
        d.group_size = static_cast<std::int32_t>(spec.attributes[1]);
        d.rows = W.size(0);
        d.cols = x.size(-1);
        d.values = W.data();
        d.values_dtype = kq_dtype_of(W.dtype());
        d.scales = S.data();
        d.scales_dtype = kq_dtype_of(S.dtype());
        d.zeros = nullptr;
        d.zeros_dtype = KQ_NONE;
        if (in.size() == 4) {  // bound zero (Context::bind_packed_zero): additive F32/F16, or uint4 zero points as U8
            d.zeros = in[3].data();
            d.zeros_dtype = in[3].dtype() == DType::U8 ? KQ_ZP_U8 : kq_dtype_of(in[3].dtype());
        }
        d.memory = on_device ? KQ_DEVICE : KQ_HOST;
        if (const kq_status s = kq_weight_pack(&d, stream_, &weight_); s != KQ_OK) raise(s);
        input_scale_ = spec.epsilon;  // 0 = dynamic activations
        output_scale_ = std::bit_cast<float>(static_cast<std::int32_t>(spec.attributes[2]));
        rows_ = d.rows;
        cols_ = d.cols;
    }
    ~PackedLinear() override { kq_weight_free(weight_); }
    PackedLinear(const PackedLinear&) = delete;
    PackedLinear& operator=(const PackedLinear&) = delete;

    auto run(TensorInputs in) -> Tensor override {
        check_input(in);
        auto shape = in[0].shape_vector();
        shape.back() = rows_;
        std::array<Tensor, 1> out{pool_.acquire(shape, DType::F32, in[0].device())};
        run_into(in, out);
        return out[0];
    }
    auto run_(TensorInputs, Tensor&) -> Tensor override {
        ops::fail(ErrorCode::UNSUPPORTED, "packed linear cannot run in place");  // as runtime/ynn/operators.cpp:1256
    }
    auto run_into(TensorInputs in, std::span<Tensor> outputs) -> void override {
        check_input(in);
        if (outputs.empty()) ops::fail(ErrorCode::INVALID_ARGUMENT, "packed linear needs one output");
        Tensor& y = outputs.back();
        const Tensor& x = in[0];
        const std::int64_t m = x.element_count() / cols_;
        if (y.dtype() != DType::F32 || y.dimensions() == 0 || y.size(-1) != rows_ || y.element_count() != m * rows_)
            ops::fail(ErrorCode::INVALID_ARGUMENT, "packed linear output shape or dtype mismatch");
        const bool direct = x.device() == device_ && y.device() == device_;
        Tensor xd = x, yd = y;
        if (!direct) {  // a CPU-device graph: stage through device buffers kept for reuse
            xd = staging_.acquire(x.shape(), x.dtype(), device_);
            yd = staging_.acquire(y.shape(), DType::F32, device_);
            if (x.device() != device_) copy_tensor(xd, x);
            else xd = x;
        }
        kq_linear_args a{};
        a.x = xd.data();
        a.x_dtype = kq_dtype_of(x.dtype());
        a.m = m;
        a.input_scale = input_scale_;
        a.output_scale = output_scale_;
        a.y = static_cast<float*>(yd.data());
        if (const kq_status s = kq_packed_linear(weight_, &a, stream_); s != KQ_OK) raise(s);
        if (!direct) {
            if (const hipError_t e = hipStreamSynchronize(stream_); e != hipSuccess)
                ops::fail(ErrorCode::RUNTIME, std::string("hipStreamSynchronize failed: ") + hipGetErrorString(e));
            copy_tensor(y, yd);
        }
    }
    auto allocations() const -> AllocationStats override { return pool_.allocations(); }
    auto release_workspaces() -> void override { staging_.clear(); }

private:
    void check_input(const TensorInputs& in) const {
        if (in.size() == 0 || in[0].dimensions() == 0 || in[0].size(-1) != cols_ ||
            (in[0].dtype() != DType::F32 && in[0].dtype() != DType::BF16))
            ops::fail(ErrorCode::INVALID_ARGUMENT, "packed linear shape or dtype mismatch");
    }

    kq_weight* weight_ = nullptr;
    hipStream_t stream_;
    tensor::Device device_;  // the HIP device of the weight and the staging buffers
    float input_scale_ = 0, output_scale_ = 0;
    std::int64_t rows_ = 0, cols_ = 0;
    OutputPool pool_;
    OutputPool staging_;
};

class Compiler final : public graph::Compiler {
public:
    Compiler(hipStream_t stream, tensor::Device device) : stream_(stream), device_(device) {}
    auto name() const -> std::string_view override { return "hip"; }
    auto prepare_operator(const OperatorSpec& spec, TensorInputs in) -> std::unique_ptr<Operator> override {
        if (spec.operation != Operation::PACKED_LINEAR) return nullptr;  // decline: the backend handles it
        return std::make_unique<PackedLinear>(spec, in, stream_, device_);
    }

private:
    hipStream_t stream_;
    tensor::Device device_;
};

class HipOperators final : public OperatorBackend {
public:
    HipOperators(tensor::Device device, hipStream_t stream)
        : device_(device), stream_(stream), compiler_(std::make_shared<Compiler>(stream, device)) {}
    auto prepare(const OperatorSpec& spec, TensorInputs in) -> std::unique_ptr<Operator> override {
        if (spec.operation == Operation::PACKED_LINEAR) return std::make_unique<PackedLinear>(spec, in, stream_, device_);
        ops::fail(ErrorCode::UNSUPPORTED, std::string("operation ") + std::string(operation_name(spec.operation)) +
                                              " is not supported by the HIP backend");
    }
    auto synchronize() -> void override {
        if (const hipError_t e = hipStreamSynchronize(stream_); e != hipSuccess)
            ops::fail(ErrorCode::RUNTIME, std::string("hipStreamSynchronize failed: ") + hipGetErrorString(e));
    }
    auto supports_replay() const noexcept -> bool override { return true; }  // PackedLinear implements run_into
    auto graph_compiler() -> std::shared_ptr<graph::Compiler> override { return compiler_; }
    auto copy_slice_(Tensor&, const Tensor&, std::size_t, std::size_t, std::size_t, std::size_t) -> void override {
        ops::fail(ErrorCode::UNSUPPORTED, "copy_slice_ is not supported by the HIP backend");
    }

private:
    tensor::Device device_;
    hipStream_t stream_;
    std::shared_ptr<Compiler> compiler_;
};

auto hip_operators(tensor::Device device, hipStream_t stream) -> std::unique_ptr<OperatorBackend> {
    return std::make_unique<HipOperators>(device, stream);
}

}  // namespace kidi::runtime::hip

// ---------------------------------------------------------------------------------------------------------------
// Test surface (no counterpart in Kidi): the adapter driven through raw pointers.

namespace {
using namespace kidi;
thread_local std::string g_error;

int status_of(const ops::Failure& f) {
    g_error = f.error().message;
    return static_cast<int>(f.error().code) + 1;
}
tensor::DType dtype_from(int kq) {
    switch (kq) {
        case KQ_F32: return tensor::DType::F32;
        case KQ_F16: return tensor::DType::F16;
        case KQ_BF16: return tensor::DType::BF16;
        case KQ_I8: return tensor::DType::I8;
        default: return tensor::DType::U8;  // KQ_U8, KQ_ZP_U8
    }
}
tensor::Device device_from(int on_device) {
    int dev = 0;
    if (on_device) (void)hipGetDevice(&dev);
    return {on_device ? tensor::DeviceKind::HIP : tensor::DeviceKind::CPU, dev};
}
}  // namespace

struct kqa_op {
    std::unique_ptr<runtime::OperatorBackend> backend;
    std::unique_ptr<runtime::Operator> op;
    tensor::Tensor held;  // a run() result the caller keeps (its storage is then not unique)
};

extern "C" {

const char* kqa_last_error(void) { return g_error.c_str(); }

const char* kqa_operation_name(int operation) {
    try {
        static thread_local std::string name;
        name = std::string(runtime::operation_name(static_cast<runtime::Operation>(operation)));
        return name.c_str();
    } catch (const std::out_of_range&) {
        return nullptr;
    }
}

// Prepares PACKED_LINEAR for a weight described as in kq_pack_desc (d->cols = K) through the graph::Compiler
// interceptor (via_backend = 0) or OperatorBackend::prepare (1).
int kqa_prepare(const kq_pack_desc* d, float input_scale, float output_scale, int via_backend, void* stream, kqa_op** out) {
    try {
        if (!d || !out) ops::fail(core::ErrorCode::INVALID_ARGUMENT, "null argument");
        const tensor::Device dev = device_from(d->memory == KQ_DEVICE);
        const int per_byte = (d->bits == 2 || d->bits == 4 || d->bits == 8) ? 8 / d->bits : 1;
        const std::int64_t groups = d->group_size > 0 ? d->cols / d->group_size : 0;
        const auto x_proto = tensor::Tensor::borrow(nullptr, {1, d->cols}, tensor::DType::F32, dev);
        const auto W = tensor::Tensor::borrow(const_cast<void*>(d->values), {d->rows, d->cols / per_byte}, dtype_from(d->values_dtype), dev);
        const auto S = tensor::Tensor::borrow(const_cast<void*>(d->scales), {d->rows, groups}, dtype_from(d->scales_dtype), dev);
        const auto Z = tensor::Tensor::borrow(const_cast<void*>(d->zeros), {d->rows, groups}, dtype_from(d->zeros_dtype), dev);
        const std::array<std::int64_t, 3> attributes{d->bits, d->group_size, std::bit_cast<std::int32_t>(output_scale)};
        const runtime::OperatorSpec spec{runtime::Operation::PACKED_LINEAR, attributes, tensor::DType::F32, input_scale};
        auto h = std::make_unique<kqa_op>();
        h->backend = runtime::hip::hip_operators(dev, static_cast<hipStream_t>(stream));
        const bool zeros = d->zeros != nullptr;
        if (via_backend) {
            h->op = zeros ? h->backend->prepare(spec, {&x_proto, &W, &S, &Z}) : h->backend->prepare(spec, {&x_proto, &W, &S});
        } else {
            auto compiler = h->backend->graph_compiler();
            h->op = zeros ? compiler->prepare_operator(spec, {&x_proto, &W, &S, &Z}) : compiler->prepare_operator(spec, {&x_proto, &W, &S});
        }
        *out = h.release();
        return 0;
    } catch (const ops::Failure& f) {
        return status_of(f);
    }
}

// Another operation through the interceptor (1: declined, the backend would run it) or the backend (its status).
int kqa_prepare_other(int operation, int via_backend) {
    try {
        const std::array<std::int64_t, 1> attributes{0};
        const runtime::OperatorSpec spec{static_cast<runtime::Operation>(operation), attributes};
        auto backend = runtime::hip::hip_operators(device_from(0), nullptr);
        const auto x = tensor::Tensor::borrow(nullptr, {1, 1}, tensor::DType::F32, device_from(0));
        if (!via_backend) return backend->graph_compiler()->prepare_operator(spec, {&x}) ? 0 : -1;
        return backend->prepare(spec, {&x}) ? 0 : -2;
    } catch (const ops::Failure& f) {
        return status_of(f);
    }
}

// run(): *y receives the pool tensor's data (owned by the operator); hold = 1 keeps the result alive here, as a
// caller that still uses it would.
int kqa_run(kqa_op* h, const void* x, int x_dtype, int64_t m, int64_t cols, int on_device, int hold, void** y) {
    try {
        const auto xt = tensor::Tensor::borrow(const_cast<void*>(x), {m, cols}, dtype_from(x_dtype), device_from(on_device));
        tensor::Tensor out = h->op->run({&xt});
        *y = out.data();
        if (hold) h->held = out;
        return 0;
    } catch (const ops::Failure& f) {
        return status_of(f);
    }
}

int kqa_run_into(kqa_op* h, const void* x, int x_dtype, int64_t m, int64_t cols, float* y, int64_t y_rows, int64_t y_cols,
                 int on_device) {
    try {
        const tensor::Device dev = device_from(on_device);
        const auto xt = tensor::Tensor::borrow(const_cast<void*>(x), {m, cols}, dtype_from(x_dtype), dev);
        std::array<tensor::Tensor, 1> outs{tensor::Tensor::borrow(y, {y_rows, y_cols}, tensor::DType::F32, dev)};
        h->op->run_into({&xt}, outs);
        return 0;
    } catch (const ops::Failure& f) {
        return status_of(f);
    }
}

int kqa_run_(kqa_op* h, const void* x, int x_dtype, int64_t m, int64_t cols, float* y, int64_t y_cols, int on_device) {
    try {
        const tensor::Device dev = device_from(on_device);
        const auto xt = tensor::Tensor::borrow(const_cast<void*>(x), {m, cols}, dtype_from(x_dtype), dev);
        auto dst = tensor::Tensor::borrow(y, {m, y_cols}, tensor::DType::F32, dev);
        (void)h->op->run_({&xt}, dst);
        return 0;
    } catch (const ops::Failure& f) {
        return status_of(f);
    }
}

int kqa_synchronize(kqa_op* h) {
    try {
        h->backend->synchronize();
        return 0;
    } catch (const ops::Failure& f) {
        return status_of(f);
    }
}

void kqa_allocations(const kqa_op* h, uint64_t* count, uint64_t* bytes) {
    const auto a = h->op->allocations();
    *count = a.count;
    *bytes = a.bytes;
}

int kqa_supports_replay(const kqa_op* h) { return h->backend->supports_replay() ? 1 : 0; }

void kqa_release(kqa_op* h) { h->held = tensor::Tensor{}; }

void kqa_free(kqa_op* h) { delete h; }

}  // extern "C"
