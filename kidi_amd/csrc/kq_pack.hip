// Load-time weight quantization on the device: Kidi's ops::pack_weight (src/kidi/ops/quantization.cpp:12-133), the
// packing Context::prepare_linear_weights runs for float weights (ops/context.cpp:783-812). Float weights [rows, width]
// (F32, F16 or BF16) become Kidi-layout packed codes U8 [rows, width / (8 / bits)] (element k in bits
// (k % (8/bits)) * bits of byte k / (8/bits), two's complement), F32 scales [rows, width / g] and, for the 4-bit
// asymmetric clip, F32 additive zeros [rows, width / g]:
//   symmetric: scale = max|w| / limit (1 when max = 0), c = clamp(round-half-away(w / scale), -limit, limit),
//              limit = 2^(bits-1) - 1 (round half away from zero decided on the remainder after truncation, :37-44);
//   asymmetric 4-bit (:49-93): for frac in 1.00, 0.95, ..., 0.50: sc = max(2 frac half / 15, 1e-8),
//              zp = clamp(rint(-(center - frac half) / sc), 0, 15), mse = sum (w - (clamp(rint(w / sc + zp), 0, 15) -
//              zp) sc)^2 in channel order; the first minimum wins (strict <); c = q - 8, zero = (8 - zp) sc.
// One thread per (row, group) walks its group in channel order, so every float operation happens in the reference's
// order (-ffp-contract=off keeps each a*b+c two roundings). A group covers whole bytes (g % (8/bits) == 0), so no byte
// is shared between threads. Non-finite weights and a symmetric scale that underflows to 0 set an error flag
// (INVALID_ARGUMENT in the reference).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kq_internal.hpp"

namespace kq {
namespace {

struct PackArgs {
    const void* w;
    int dtype;  // 0 F32, 1 F16, 2 BF16
    std::int64_t rows, width, group;
    int bits, asym;
    std::uint8_t* values;
    float* scales;
    float* zeros;
    int* error;  // 1: non-finite weight, 2: scale underflow
};

__device__ __forceinline__ float read_w(const PackArgs& a, std::int64_t i) {
    if (a.dtype == 0) return static_cast<const float*>(a.w)[i];
    const std::uint16_t h = static_cast<const std::uint16_t*>(a.w)[i];
    if (a.dtype == 1) return __half2float(__ushort_as_half(h));
    return __uint_as_float(static_cast<std::uint32_t>(h) << 16);
}

__global__ __launch_bounds__(256) void pack_weight_kernel(PackArgs a) {
    const std::int64_t groups = a.width / a.group;
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= a.rows * groups) return;
    const std::int64_t row = id / groups, grp = id - row * groups;
    const std::int64_t begin = row * a.width + grp * a.group;
    const int per = 8 / a.bits;
    const int limit = (1 << (a.bits - 1)) - 1;
    std::uint8_t* out = a.values + begin / per;  // the group's bytes (whole bytes)
    if (a.asym) {
        float mn = __builtin_inff(), mx = -__builtin_inff();
        bool finite = true;
        for (std::int64_t c = 0; c < a.group; ++c) {
            const float v = read_w(a, begin + c);
            finite &= __builtin_isfinite(v);
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        if (!finite) {
            atomicOr(a.error, 1);
            return;
        }
        const float center = 0.5F * (mx + mn);
        const float half = 0.5F * (mx - mn);
        float best_scale = 1.F, best_zp = 8.F, best_mse = __builtin_inff();
        const float fractions[11] = {1.00F, 0.95F, 0.90F, 0.85F, 0.80F, 0.75F, 0.70F, 0.65F, 0.60F, 0.55F, 0.50F};
        for (int f = 0; f < 11; ++f) {
            const float frac = fractions[f];
            const float lo = center - frac * half;
            const float sc = fmaxf((2.0F * frac * half) / 15.0F, 1e-8F);
            const float zp = fminf(fmaxf(__builtin_rintf(-lo / sc), 0.0F), 15.0F);
            float mse = 0.0F;
            for (std::int64_t c = 0; c < a.group; ++c) {
                const float w = read_w(a, begin + c);
                const float q = fminf(fmaxf(__builtin_rintf(w / sc + zp), 0.0F), 15.0F);
                const float diff = w - (q - zp) * sc;
                mse += diff * diff;
            }
            if (mse < best_mse) {
                best_mse = mse;
                best_scale = sc;
                best_zp = zp;
            }
        }
        a.scales[id] = best_scale;
        a.zeros[id] = (8.0F - best_zp) * best_scale;
        for (std::int64_t c = 0; c < a.group; c += 2) {
            std::uint32_t byte = 0;
            for (int h = 0; h < 2; ++h) {
                const float w = read_w(a, begin + c + h);
                const int q = static_cast<int>(fminf(fmaxf(__builtin_rintf(w / best_scale + best_zp), 0.0F), 15.0F));
                byte |= static_cast<std::uint32_t>((q - 8) & 0xF) << (4 * h);
            }
            out[c / 2] = static_cast<std::uint8_t>(byte);
        }
        return;
    }
    float maximum = 0.F;
    bool finite = true;
    for (std::int64_t c = 0; c < a.group; ++c) {
        const float v = read_w(a, begin + c);
        finite &= __builtin_isfinite(v);
        maximum = fmaxf(maximum, fabsf(v));
    }
    if (!finite) {
        atomicOr(a.error, 1);
        return;
    }
    const float scale = maximum == 0.F ? 1.F : maximum / static_cast<float>(limit);
    if (scale == 0.F) {
        atomicOr(a.error, 2);
        return;
    }
    a.scales[id] = scale;
    for (std::int64_t c = 0; c < a.group; c += per) {
        std::uint32_t byte = 0;
        for (int i = 0; i < per; ++i) {
            const float quotient = read_w(a, begin + c + i) / scale;
            float rounded = truncf(quotient);
            if (fabsf(quotient - rounded) >= 0.5F) rounded += copysignf(1.F, quotient);
            const int code = static_cast<int>(fminf(fmaxf(rounded, -static_cast<float>(limit)), static_cast<float>(limit)));
            byte |= static_cast<std::uint32_t>(code & ((1 << a.bits) - 1)) << (i * a.bits);
        }
        out[c / per] = static_cast<std::uint8_t>(byte);
    }
}

}  // namespace

hipError_t launch_pack_weight(const void* w, int dtype, std::int64_t rows, std::int64_t width, int bits, std::int64_t group,
                              bool asym, std::uint8_t* values, float* scales, float* zeros, int* error, hipStream_t stream) {
    PackArgs a{};
    a.w = w;
    a.dtype = dtype;
    a.rows = rows;
    a.width = width;
    a.group = group;
    a.bits = bits;
    a.asym = asym ? 1 : 0;
    a.values = values;
    a.scales = scales;
    a.zeros = zeros;
    a.error = error;
    const std::int64_t n = rows * (width / group);
    hipLaunchKernelGGL(pack_weight_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace kq
