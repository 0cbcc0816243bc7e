// kq_ref — CPU oracle for Kidi's PACKED_LINEAR operator.
//
// TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
// library, and only as the checker (or as the timed CPU baseline). The product path (kidi_amd/) never calls it.
//
// Kidi's own CPU arithmetic for this operator lives in the third_party/ynnpack-dev submodule (pin
// 2f503485e2e5ea0e3cd29d7ca5b5223d0699cfc0, recorded at benchmarks/cpu/reference.json:268), which is absent from
// the reference checkout, and Kidi's C++ needs <expected>, which this toolchain lacks. Every function below is
// therefore a restatement of a closed form that the reference pins in readable source or tests; each cites it.
//
// Pinning status (what checks each function; the tests live in tests/test_oracle_*.py):
//   kqr_pack_weight         pinned: quantization.cpp closed form + arm_gemma_benchmark_test.py:83-101 KATs +
//                           eager_test.cpp:300-331 layout/decode + invariants (round trip, argmin by brute force).
//   kqr_unpack_codes        pinned: eager_test.cpp:318-320, precision_test.cpp:95-108 (0xe1,0xc3 -> -5).
//   kqr_qat_to_signed       pinned: closed form model/gemma4.cpp:358-369 + round-trip identity.
//   kqr_quantize_static     pinned: eager_test.cpp:94-103 exact KAT, vulkan/operators.cpp:809-826.
//   kqr_quantize_dynamic    partially pinned: hnsw_test.cpp:490-520 restates it for the HNSW search; that
//                           ynn::quantize_blockwise_blocks_f32 is byte-identical is presumed, not proven. The
//                           all-zero block (undefined there: 0*inf) is defined here as codes 0, scale 0.
//   kqr_partials            pinned by brute force (int64 double loop) and closed form; order-independent.
//   kqr_packed_linear       static (calibrated) path pinned exactly by eager_test.cpp:64-111 and the CUDA KAT
//                           tests/kidi/runtime/cuda/operators_test.cpp:815-831; dynamic BlockwiseLinear path is
//                           PARITY UNPINNED beyond its closed form (no reference test hits it with a tight
//                           expected value); portable float path pinned to 1e-3 / 0.05 by eager_test.cpp:300-378.
//   kqr_gelu_tanh           pinned by eager_test.cpp:431-452 (formula to 1e-5 and exact saturation values).
//   kqr_silu_gate           pinned by eager_test.cpp:167-186 (g / (1 + exp(-g)) * up to 1e-5).
//   kqr_parity_linear       pinned: precision_test.cpp:87-92 LOWBIT_PARITY KAT (exact outputs 0.4, 0) and the
//                           reference's own cross-check graph_test.cpp:158-177 (LOWBIT_PARITY within 1e-5 of the
//                           calibrated SymmetricPackedLinear path); bit-exact to parity_math.cpp for M < 8 (serial
//                           FMA), while for M >= 8 the reference sums with Accelerate's sgemm, whose order is unknown.
//   kqr_rms_norm            pinned: eager_test.cpp:388-412 KAT (plain, 2x weight, residual, scaled; zero row
//                           exactly 0), cuda/operators_test.cpp:346-350 identity (residual form == (norm + r) * s
//                           exactly), float64 closed form to a few ulp, power-of-two weight scaling exact. The
//                           summation order of the sum of squares is this build's definition (Kidi's
//                           ynn::rms_norm_f32 order is unknown); the GPU paths follow the same order.
//
// Floating point: compiled with -ffp-contract=off so every a*b+c rounds twice, as ISO C++ evaluation does.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

enum DType : int { F32 = 0, F16 = 1, BF16 = 2, U8 = 3, I8 = 4, ZP_U8 = 5 };

// IEEE-754 binary16 -> binary32, exact for every input (normals, subnormals, inf, NaN), written from the format
// definition. Kidi uses an exact conversion too (checkpoint/ggml/dequantize.h:45-58); any exact one agrees.
float half_to_float(std::uint16_t h) {
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const std::uint32_t exponent = (h >> 10) & 0x1fu;
    std::uint32_t mantissa = h & 0x3ffu;
    std::uint32_t bits;
    if (exponent == 0x1fu) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;
    } else {
        // Subnormal half: value = mantissa * 2^-24. Normalise into a float.
        int shift = 0;
        while ((mantissa & 0x400u) == 0) {
            mantissa <<= 1;
            ++shift;
        }
        mantissa &= 0x3ffu;
        bits = sign | (static_cast<std::uint32_t>(113 - shift) << 23) | (mantissa << 13);
    }
    float out;
    std::memcpy(&out, &bits, sizeof out);
    return out;
}

float bf16_to_float(std::uint16_t b) {
    const std::uint32_t bits = static_cast<std::uint32_t>(b) << 16;
    float out;
    std::memcpy(&out, &bits, sizeof out);
    return out;
}

float load_float(const void* base, int dtype, std::size_t index) {
    switch (dtype) {
    case F32: return static_cast<const float*>(base)[index];
    case F16: return half_to_float(static_cast<const std::uint16_t*>(base)[index]);
    case BF16: return bf16_to_float(static_cast<const std::uint16_t*>(base)[index]);
    default: return std::numeric_limits<float>::quiet_NaN();
    }
}

// Signed code of element k of a packed row: ((byte >> bits*(k mod 8/bits)) & mask) ^ sign) - sign.
// eager_test.cpp:318-320 (`(raw ^ (1 << (bits - 1))) - (1 << (bits - 1))`), low bits hold the even element
// (ops/quantization.cpp:91, :113-114).
int code_at(const std::uint8_t* row, int bits, std::int64_t k) {
    if (bits == 8) return static_cast<std::int8_t>(row[k]);
    const int per_byte = 8 / bits;
    const int raw = (row[k / per_byte] >> ((k % per_byte) * bits)) & ((1 << bits) - 1);
    const int sign = 1 << (bits - 1);
    return (raw ^ sign) - sign;
}

float clampf(float v, float lo, float hi) { return std::min(std::max(v, lo), hi); }

struct Linear {
    const float* x;
    std::int64_t M, K, N;
    const std::uint8_t* values;
    int bits, group;
    const void* scales;
    int scales_dtype;
    const void* zeros;
    int zeros_dtype;  // -1: none; F32/F16: additive zero; ZP_U8: one zero-point byte per group
    float input_scale, output_scale;
    float* y;
};

float zero_at(const Linear& p, std::size_t index, float scale) {
    if (p.zeros_dtype == ZP_U8) return (8.0F - static_cast<float>(static_cast<const std::uint8_t*>(p.zeros)[index])) * scale;
    return load_float(p.zeros, p.zeros_dtype, index);
}

float calibrate_output(float value, float output_scale) {
    // Static output rounding, eager_test.cpp:100-102; quantized_linear.metal:150-153 (rint).
    if (output_scale > 0.F) return clampf(std::nearbyint(value / output_scale), -128.F, 127.F) * output_scale;
    return value;
}

// Which CPU operator Kidi selects for PACKED_LINEAR, runtime/ynn/operators.cpp:2739-2900 (selection order),
// BlockwiseLinear::supports :1038-1059, SymmetricPackedLinear::supports :1185-1204.
enum Path : int { PATH_BLOCKWISE = 0, PATH_SYMMETRIC = 1, PATH_PORTABLE = 2 };

int select_path(int bits, std::int64_t group, std::int64_t K, std::int64_t N, bool has_zero, float input_scale) {
    if (input_scale <= 0.F) {
        bool blockwise = group >= 32 && K % group == 0;
        if (blockwise && bits == 4) blockwise = group % 32 == 0 && (has_zero || (group < K && N >= 256));
        else if (blockwise && bits == 8) blockwise = group % 16 == 0 && !has_zero && N >= 64;
        else blockwise = false;
        if (blockwise) return PATH_BLOCKWISE;
    } else if (!has_zero && group > 0 && K % group == 0 && group % (8 / bits) == 0) {
        return PATH_SYMMETRIC;
    }
    return PATH_PORTABLE;
}

}  // namespace

extern "C" {

int kqr_select_path(int bits, std::int64_t group, std::int64_t K, std::int64_t N, int has_zero, float input_scale) {
    return select_path(bits, group, K, N, has_zero != 0, input_scale);
}

float kqr_half_to_float(std::uint16_t h) { return half_to_float(h); }

// ops::pack_weight, src/kidi/ops/quantization.cpp:12-133. `weight` is [rows, width] in F32/F16/BF16.
// Outputs: values U8 [rows, width/(8/bits)] (zero-filled then OR-ed, :22-23), scales F32 [rows, width/group],
// zeros F32 [rows, width/group] for the 4-bit asymmetric clip (`(8 - zp) * scale`, :85). Returns 0, or 1 for
// INVALID_ARGUMENT (bad shape/bits/group :15-20, non-finite weight :59-60/:102, scale underflow :104).
int kqr_pack_weight(const void* weight, int dtype, std::int64_t rows, std::int64_t width, int bits,
                    std::int64_t group, int asymmetric_clip, std::uint8_t* values, float* scales, float* zeros) {
    if ((dtype != F32 && dtype != F16 && dtype != BF16) || (bits != 2 && bits != 4 && bits != 8) || group <= 0 ||
        group % (8 / bits) || rows <= 0 || width <= 0 || width % group)
        return 1;
    const std::int64_t groups = width / group;
    const std::int64_t per_byte = 8 / bits;
    const int limit = (1 << (bits - 1)) - 1;
    const bool asym = asymmetric_clip != 0 && bits == 4;
    std::memset(values, 0, static_cast<std::size_t>(rows * (width / per_byte)));
    // Round half away from zero after exact truncation, :37-44.
    const auto quantize = [&](float value, float scale) {
        const float quotient = value / scale;
        float rounded = std::trunc(quotient);
        if (std::fabs(quotient - rounded) >= 0.5F) rounded += std::copysign(1.F, quotient);
        return static_cast<int>(clampf(rounded, -static_cast<float>(limit), static_cast<float>(limit)));
    };
    static const float fractions[11] = {1.00F, 0.95F, 0.90F, 0.85F, 0.80F, 0.75F,
                                        0.70F, 0.65F, 0.60F, 0.55F, 0.50F};  // :65-66
    for (std::int64_t row = 0; row < rows; ++row) {
        for (std::int64_t g = 0; g < groups; ++g) {
            const std::int64_t begin = row * width + g * group;
            const auto read = [&](std::int64_t c) { return load_float(weight, dtype, static_cast<std::size_t>(begin + c)); };
            if (asym) {
                // 11-step MSE clip search, :49-93.
                float mn = std::numeric_limits<float>::infinity();
                float mx = -std::numeric_limits<float>::infinity();
                bool finite = true;
                for (std::int64_t c = 0; c < group; ++c) {
                    const float v = read(c);
                    finite = finite && std::isfinite(v);
                    mn = std::min(mn, v);
                    mx = std::max(mx, v);
                }
                if (!finite) return 1;
                const float center = 0.5F * (mx + mn);
                const float half = 0.5F * (mx - mn);
                float best_scale = 1.F, best_zp = 8.F, best_mse = std::numeric_limits<float>::infinity();
                for (const float frac : fractions) {
                    const float lo = center - frac * half;
                    const float sc = std::max((2.0F * frac * half) / 15.0F, 1e-8F);
                    const float zp = clampf(std::nearbyint(-lo / sc), 0.0F, 15.0F);
                    float mse = 0.0F;
                    for (std::int64_t c = 0; c < group; ++c) {
                        const float w = read(c);
                        const float q = clampf(std::nearbyint(w / sc + zp), 0.0F, 15.0F);
                        const float diff = w - (q - zp) * sc;
                        mse += diff * diff;
                    }
                    if (mse < best_mse) {  // strict: the first of equal errors wins (:78)
                        best_mse = mse;
                        best_scale = sc;
                        best_zp = zp;
                    }
                }
                scales[row * groups + g] = best_scale;
                zeros[row * groups + g] = (8.0F - best_zp) * best_scale;
                for (std::int64_t c = 0; c < group; ++c) {
                    const std::int64_t offset = begin + c;
                    const int q = static_cast<int>(clampf(std::nearbyint(read(c) / best_scale + best_zp), 0.0F, 15.0F));
                    values[offset / 2] |= static_cast<std::uint8_t>(((q - 8) & 0xF) << ((offset % 2) * 4));
                }
                continue;
            }
            float maximum = 0.F;
            bool finite = true;
            for (std::int64_t c = 0; c < group; ++c) {
                const float v = read(c);
                finite = finite && std::isfinite(v);
                maximum = std::max(maximum, std::fabs(v));
            }
            if (!finite) return 1;
            const float scale = maximum == 0.F ? 1.F : maximum / static_cast<float>(limit);  // :103
            if (scale == 0.F) return 1;
            scales[row * groups + g] = scale;
            for (std::int64_t c = 0; c < group; ++c) {
                const std::int64_t offset = begin + c;
                const int q = quantize(read(c), scale);
                if (bits == 8) values[offset] = static_cast<std::uint8_t>(q);
                else values[offset / per_byte] |= static_cast<std::uint8_t>((q & ((1 << bits) - 1)) << ((offset % per_byte) * bits));
            }
        }
    }
    return 0;
}

// Signed codes [rows, width] from packed values (see code_at).
int kqr_unpack_codes(const std::uint8_t* values, std::int64_t rows, std::int64_t width, int bits, std::int8_t* codes) {
    if (bits != 2 && bits != 4 && bits != 8) return 1;
    const std::int64_t row_bytes = width / (8 / bits);
    for (std::int64_t r = 0; r < rows; ++r)
        for (std::int64_t k = 0; k < width; ++k)
            codes[r * width + k] = static_cast<std::int8_t>(code_at(values + r * row_bytes, bits, k));
    return 0;
}

// QAT checkpoint conversion, src/kidi/model/gemma4.cpp:358-369: offset-binary codes -> two's complement nibbles
// (XOR 0x88) or crumbs (XOR 0xaa); 8-bit bytes are left untouched.
void kqr_qat_to_signed(std::uint8_t* bytes, std::int64_t count, int bits) {
    if (bits >= 8) return;
    const std::uint8_t mask = bits == 2 ? 0xaa : 0x88;
    for (std::int64_t i = 0; i < count; ++i) bytes[i] ^= mask;
}

// Dynamic per-(row, block) activation quantization used by BlockwiseLinear (operators.cpp:1118-1126), restated
// from tests/kidi/search/hnsw_test.cpp:490-520.
//  bits 2/4 (symmetric): max = max|x|, scale = max/127, inverse = 127/max, q = clamp(nearbyint(x*inverse), -127, 127);
//    an all-zero block gives codes 0 and scale 0.
//  bits 8 (asymmetric, :492-511): rmin = min(0, x), rmax = max(0, x), inverse = 255/(rmax-rmin),
//    scale = (rmax-rmin)/255, zp = rint(clamp(fzp, -128, 127)), q = clamp(round(x*inverse) + zp, -128, 127)
//    (std::round: ties away from zero); an all-zero block gives inverse 0, scale 1, zp -128.
// Outputs q [M, K], scale [M, K/group], sum [M, K/group] (sum of q over the block), zero_point [M, K/group]
// (0 for the symmetric form).
int kqr_quantize_dynamic(const float* x, std::int64_t M, std::int64_t K, std::int64_t group, int bits,
                         std::int8_t* q, float* scale, std::int32_t* sum, std::int32_t* zero_point) {
    if (group <= 0 || K % group) return 1;
    const std::int64_t blocks = K / group;
    for (std::int64_t m = 0; m < M; ++m)
        for (std::int64_t b = 0; b < blocks; ++b) {
            const float* xb = x + m * K + b * group;
            std::int8_t* qb = q + m * K + b * group;
            std::int32_t total = 0;
            if (bits == 8) {
                float rmin = 0.F, rmax = 0.F;
                for (std::int64_t c = 0; c < group; ++c) {
                    rmin = std::min(rmin, xb[c]);
                    rmax = std::max(rmax, xb[c]);
                }
                const float rdiff = rmax - rmin;
                const float inverse = rdiff > 0.F ? 255.F / rdiff : 0.F;
                const float s = rdiff > 0.F ? rdiff / 255.F : 1.F;
                const float min_error = -128.F + rmin * inverse;
                const float max_error = 127.F + rmax * inverse;
                const float fzp = min_error + max_error > 0.F ? -128.F - rmin * inverse : 127.F - rmax * inverse;
                const std::int32_t zp = rdiff > 0.F ? static_cast<std::int32_t>(std::rint(clampf(fzp, -128.F, 127.F))) : -128;
                for (std::int64_t c = 0; c < group; ++c) {
                    const std::int32_t v = std::clamp<std::int32_t>(static_cast<std::int32_t>(std::round(xb[c] * inverse)) + zp, -128, 127);
                    qb[c] = static_cast<std::int8_t>(v);
                    total += v;
                }
                scale[m * blocks + b] = s;
                zero_point[m * blocks + b] = zp;
            } else {
                float maximum = 0.F;
                for (std::int64_t c = 0; c < group; ++c) maximum = std::max(maximum, std::fabs(xb[c]));
                if (maximum == 0.F) {
                    for (std::int64_t c = 0; c < group; ++c) qb[c] = 0;
                    scale[m * blocks + b] = 0.F;
                } else {
                    const float inverse = 127.F / maximum;
                    for (std::int64_t c = 0; c < group; ++c) {
                        const std::int32_t v = static_cast<std::int32_t>(clampf(std::nearbyint(xb[c] * inverse), -127.F, 127.F));
                        qb[c] = static_cast<std::int8_t>(v);
                        total += v;
                    }
                    scale[m * blocks + b] = maximum / 127.F;
                }
                zero_point[m * blocks + b] = 0;
            }
            sum[m * blocks + b] = total;
        }
    return 0;
}

// Static (calibrated) activation quantization, SymmetricPackedLinear (operators.cpp:1183-1319) as pinned by
// eager_test.cpp:97-98 and vulkan/operators.cpp:818-819: q = clamp(nearbyint(x / input_scale), -128, 127).
int kqr_quantize_static(const float* x, std::int64_t M, std::int64_t K, std::int64_t group, float input_scale,
                        std::int8_t* q, std::int32_t* sum) {
    if (group <= 0 || K % group || !(input_scale > 0.F)) return 1;
    const std::int64_t blocks = K / group;
    for (std::int64_t m = 0; m < M; ++m)
        for (std::int64_t b = 0; b < blocks; ++b) {
            std::int32_t total = 0;
            for (std::int64_t c = 0; c < group; ++c) {
                const std::int64_t i = m * K + b * group + c;
                const auto v = static_cast<std::int32_t>(clampf(std::nearbyint(x[i] / input_scale), -128.F, 127.F));
                q[i] = static_cast<std::int8_t>(v);
                total += v;
            }
            sum[m * blocks + b] = total;
        }
    return 0;
}

// Integer per-group partials: P[m, n, b] = sum_{k in b} q[m,k] * c[n,k]; C[n, b] = sum_{k in b} c[n,k].
int kqr_partials(const std::int8_t* q, const std::int8_t* codes, std::int64_t M, std::int64_t N, std::int64_t K,
                 std::int64_t group, std::int32_t* P, std::int32_t* C) {
    if (group <= 0 || K % group) return 1;
    const std::int64_t blocks = K / group;
    for (std::int64_t n = 0; n < N; ++n)
        for (std::int64_t b = 0; b < blocks; ++b) {
            std::int32_t csum = 0;
            for (std::int64_t c = 0; c < group; ++c) csum += codes[n * K + b * group + c];
            if (C) C[n * blocks + b] = csum;
        }
    for (std::int64_t m = 0; m < M; ++m)
        for (std::int64_t n = 0; n < N; ++n)
            for (std::int64_t b = 0; b < blocks; ++b) {
                std::int32_t acc = 0;
                for (std::int64_t c = 0; c < group; ++c)
                    acc += static_cast<std::int32_t>(q[m * K + b * group + c]) * codes[n * K + b * group + c];
                P[(m * N + n) * blocks + b] = acc;
            }
    return 0;
}

}  // extern "C"

namespace {

// Rows [n0, n1) of the integer paths. Closed form (BlockwiseLinear, operators.cpp:1118-1169, :1124-1126):
//   dynamic, 2/4-bit: y = sum_b a_s[m,b] * (w_s[n,b] * P + w_z[n,b] * Q)           (w_z = 0 if no zeros)
//   dynamic, 8-bit:   y = sum_b a_s[m,b] * (w_s[n,b] * (P - zp_a[m,b] * C[n,b]))
//   static:           y = (sum_b (w_s * P + w_z * Q)) * input_scale                 (eager_test.cpp:99-101)
// then static output rounding when output_scale > 0. Sums run over b ascending in fp32.
void integer_rows(const Linear& p, bool dynamic, const std::int8_t* q, const float* a_s, const std::int32_t* Q,
                  const std::int32_t* zp_a, std::int64_t n0, std::int64_t n1) {
    const std::int64_t blocks = p.K / p.group;
    const std::int64_t row_bytes = p.K / (8 / p.bits);
    const bool asym_act = dynamic && p.bits == 8;
    std::vector<int> codes(static_cast<std::size_t>(p.K));
    for (std::int64_t n = n0; n < n1; ++n) {
        const std::uint8_t* row = p.values + n * row_bytes;
        for (std::int64_t k = 0; k < p.K; ++k) codes[static_cast<std::size_t>(k)] = code_at(row, p.bits, k);
        for (std::int64_t m = 0; m < p.M; ++m) {
            float acc = 0.F;
            for (std::int64_t b = 0; b < blocks; ++b) {
                std::int32_t P = 0, C = 0;
                for (std::int64_t c = 0; c < p.group; ++c) {
                    const int w = codes[static_cast<std::size_t>(b * p.group + c)];
                    P += static_cast<std::int32_t>(q[m * p.K + b * p.group + c]) * w;
                    C += w;
                }
                const std::size_t meta = static_cast<std::size_t>(n * blocks + b);
                const float s = load_float(p.scales, p.scales_dtype, meta);
                float t;
                if (asym_act) {
                    t = s * static_cast<float>(P - zp_a[m * blocks + b] * C);
                } else {
                    t = s * static_cast<float>(P);
                    if (p.zeros_dtype >= 0) t = t + zero_at(p, meta, s) * static_cast<float>(Q[m * blocks + b]);
                }
                acc = dynamic ? acc + a_s[m * blocks + b] * t : acc + t;
            }
            if (!dynamic) acc = acc * p.input_scale;
            p.y[m * p.N + n] = calibrate_output(acc, p.output_scale);
        }
    }
}

// PortablePackedLinearOp (operators.cpp:2639-2713): weights unpacked to codes and dequantized (c*s + z), float
// activations (statically rounded first when input_scale > 0), fp32 dot over k ascending, output rounding.
// The ynnpack body is absent; eager_test.cpp:300-378 pins it to 1e-3 (g=4) and 0.05 (g=128, N=35).
void portable_rows(const Linear& p, std::int64_t n0, std::int64_t n1) {
    const std::int64_t blocks = p.K / p.group;
    const std::int64_t row_bytes = p.K / (8 / p.bits);
    std::vector<float> w(static_cast<std::size_t>(p.K));
    std::vector<float> xr(static_cast<std::size_t>(p.M * p.K));
    for (std::int64_t i = 0; i < p.M * p.K; ++i)
        xr[static_cast<std::size_t>(i)] = p.input_scale > 0.F
            ? clampf(std::nearbyint(p.x[i] / p.input_scale), -128.F, 127.F) * p.input_scale : p.x[i];
    for (std::int64_t n = n0; n < n1; ++n) {
        for (std::int64_t k = 0; k < p.K; ++k) {
            const std::size_t meta = static_cast<std::size_t>(n * blocks + k / p.group);
            const float s = load_float(p.scales, p.scales_dtype, meta);
            float v = static_cast<float>(code_at(p.values + n * row_bytes, p.bits, k)) * s;
            if (p.zeros_dtype >= 0) v = v + zero_at(p, meta, s);
            w[static_cast<std::size_t>(k)] = v;
        }
        for (std::int64_t m = 0; m < p.M; ++m) {
            float acc = 0.F;
            for (std::int64_t k = 0; k < p.K; ++k) acc = acc + xr[static_cast<std::size_t>(m * p.K + k)] * w[static_cast<std::size_t>(k)];
            p.y[m * p.N + n] = calibrate_output(acc, p.output_scale);
        }
    }
}

template <typename Body>
void parallel_rows(std::int64_t N, int threads, Body body) {
    if (threads <= 1 || N < 2) {
        body(0, N);
        return;
    }
    std::vector<std::thread> pool;
    const std::int64_t chunk = (N + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        const std::int64_t a = t * chunk, b = std::min(N, a + chunk);
        if (a < b) pool.emplace_back(body, a, b);
    }
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

// Context::packed_linear -> CpuBackend::prepare -> Operator::run for PACKED_LINEAR (ops/context.cpp:821-939,
// runtime/ynn/operators.cpp:2739-2900). x is F32 or BF16 [M, K]; values U8 [N, K/(8/bits)] (or I8 for 8-bit);
// scales F32/F16 [N, K/group]; zeros F32/F16 [N, K/group] additive, ZP_U8 one zero-point per group, or absent
// (zeros_dtype = -1). input_scale > 0 selects the calibrated path, output_scale > 0 the output rounding.
// Returns the path taken (0 blockwise, 1 symmetric, 2 portable) or -1 for INVALID_ARGUMENT.
int kqr_packed_linear(const void* x, int x_dtype, std::int64_t M, std::int64_t K, const std::uint8_t* values,
                      std::int64_t N, int bits, std::int64_t group, const void* scales, int scales_dtype,
                      const void* zeros, int zeros_dtype, float input_scale, float output_scale, float* y, int threads) {
    if ((bits != 2 && bits != 4 && bits != 8) || group <= 0 || K <= 0 || K % group || group % (8 / bits) || N <= 0 ||
        M < 0 || (x_dtype != F32 && x_dtype != BF16) || (scales_dtype != F32 && scales_dtype != F16) ||
        (zeros && zeros_dtype != F32 && zeros_dtype != F16 && zeros_dtype != ZP_U8) ||
        !std::isfinite(input_scale) || input_scale < 0 || !std::isfinite(output_scale) || output_scale < 0)
        return -1;
    std::vector<float> xf(static_cast<std::size_t>(M * K));
    for (std::int64_t i = 0; i < M * K; ++i) xf[static_cast<std::size_t>(i)] = load_float(x, x_dtype, static_cast<std::size_t>(i));
    Linear p{xf.data(), M, K, N, values, bits, static_cast<int>(group), scales, scales_dtype,
             zeros, zeros ? zeros_dtype : -1, input_scale, output_scale, y};
    const int path = select_path(bits, group, K, N, zeros != nullptr, input_scale);
    if (M == 0) return path;
    if (path == PATH_PORTABLE) {
        parallel_rows(N, threads, [&](std::int64_t a, std::int64_t b) { portable_rows(p, a, b); });
        return path;
    }
    const std::int64_t blocks = K / group;
    std::vector<std::int8_t> q(static_cast<std::size_t>(M * K));
    std::vector<float> a_s(static_cast<std::size_t>(M * blocks));
    std::vector<std::int32_t> Q(static_cast<std::size_t>(M * blocks)), zp(static_cast<std::size_t>(M * blocks));
    const bool dynamic = path == PATH_BLOCKWISE;
    if (dynamic) kqr_quantize_dynamic(xf.data(), M, K, group, bits, q.data(), a_s.data(), Q.data(), zp.data());
    else kqr_quantize_static(xf.data(), M, K, group, input_scale, q.data(), Q.data());
    parallel_rows(N, threads, [&](std::int64_t a, std::int64_t b) {
        integer_rows(p, dynamic, q.data(), a_s.data(), Q.data(), zp.data(), a, b);
    });
    return path;
}

// GELU with the tanh approximation, 0.5x(1 + tanh(sqrt(2/pi)(x + 0.044715x^3))) (eager_test.cpp:444-452), and the
// gated form h = gelu(gate) * up over [rows, 2*width] halves (Context::gelu_gate, ops/context.cpp:957-963).
void kqr_gelu_gate(const float* gate_up, std::int64_t rows, std::int64_t width, float* out) {
    const float k0 = 0.7978845608028654F;  // sqrt(2/pi)
    for (std::int64_t r = 0; r < rows; ++r)
        for (std::int64_t i = 0; i < width; ++i) {
            const float g = gate_up[r * 2 * width + i];
            const float u = gate_up[r * 2 * width + width + i];
            const float inner = k0 * (g + 0.044715F * g * g * g);
            out[r * width + i] = 0.5F * g * (1.F + std::tanh(inner)) * u;
        }
}

// SiLU gating h = g / (1 + exp(-g)) * up over [rows, 2*width] halves (Context::silu_gate / silu_multiply,
// ops/context.cpp:964-969; formula eager_test.cpp:176-179).
void kqr_silu_gate(const float* gate_up, std::int64_t rows, std::int64_t width, float* out) {
    for (std::int64_t r = 0; r < rows; ++r)
        for (std::int64_t i = 0; i < width; ++i) {
            const float g = gate_up[r * 2 * width + i];
            const float u = gate_up[r * 2 * width + width + i];
            out[r * width + i] = g / (1.F + std::exp(-g)) * u;
        }
}

// RMS normalization over the last axis (Context::rms_norm / rms_norm_residual, ops/context.cpp:1043-1049,
// :1103-1122; Kidi's CPU RmsNorm operator, runtime/ynn/operators.cpp:553-620, whose parity form :598-614 reads
//   inverse = 1 / sqrt(sum / width + epsilon);  y = x * inverse * weight;  residual: y = (r + x * inverse * weight)
//   [* scale]).
// The sum of squares has one fixed order: the row is cut into 512-column segments and each segment into 64
// pieces of 8 columns (columns past the width count as 0, which adds exactly nothing); a piece is summed in column
// order (s = x0*x0, s = s + x1*x1, ...), the 64 pieces of a segment pairwise as a balanced tree in piece order
// (pieces 2i and 2i+1 first, then pairs of those, ...), the segments in order.
float rms_sum_squares(const float* x, std::int64_t width) {
    float total = 0.F;
    for (std::int64_t seg = 0; seg * 512 < width; ++seg) {
        float piece[64];
        for (int l = 0; l < 64; ++l) {
            float s = 0.F;
            for (int i = 0; i < 8; ++i) {
                const std::int64_t k = seg * 512 + 8 * l + i;
                const float v = k < width ? x[k] : 0.F;
                s = i == 0 ? v * v : s + v * v;
            }
            piece[l] = s;
        }
        for (int span = 1; span < 64; span *= 2)
            for (int l = 0; l < 64; l += 2 * span) piece[l] = piece[l] + piece[l + span];
        total = seg == 0 ? piece[0] : total + piece[0];
    }
    return total;
}

// Kidi's LOWBIT_PARITY projection, runtime::parity::packed_linear (src/kidi/runtime/parity_math.cpp:226-291), reached
// from Context::packed_linear under InferencePrecision::LOWBIT_PARITY (ops/context.cpp:917-932): activations rounded
// to the calibration grid (nearbyint(x / input_scale) clamped to [-128, 127], times input_scale, :247-250), weights
// dequantized to c * s (:259-260; bound zeros are not applied in this mode), each output a serial FMA over the columns
// in order (:269-277), then the output rounded to the output_scale grid (:279-282). x F32 [M, K], values U8 Kidi
// layout, scales F32 [N, K/g], y F32 [M, N]. Returns 0; 1 (INVALID_ARGUMENT) for a non-finite or non-positive scale
// (:239-240); 2 (UNSUPPORTED) outside the domain Context::packed_linear checks (:919-929).
int kqr_parity_linear(const float* x, std::int64_t M, std::int64_t K, const std::uint8_t* values, std::int64_t N, int bits,
                      std::int64_t group, const float* scales, float input_scale, float output_scale, float* y) {
    if ((bits != 2 && bits != 4 && bits != 8) || group <= 0 || K <= 0 || K % group || group % (8 / bits) || N <= 0 ||
        M < 0 || !(input_scale > 0.F) || !(output_scale > 0.F) || !std::isfinite(input_scale) ||
        !std::isfinite(output_scale) || M > INT32_MAX || K > INT32_MAX || N > INT32_MAX)
        return 2;
    const std::int64_t B = K / group, row_bytes = K / (8 / bits);
    for (std::int64_t i = 0; i < N * B; ++i)
        if (!std::isfinite(scales[i]) || !(scales[i] > 0.F)) return 1;
    std::vector<float> xr(static_cast<std::size_t>(M * K)), w(static_cast<std::size_t>(K));
    for (std::int64_t i = 0; i < M * K; ++i) xr[static_cast<std::size_t>(i)] = clampf(std::nearbyint(x[i] / input_scale), -128.F, 127.F) * input_scale;
    for (std::int64_t n = 0; n < N; ++n) {
        for (std::int64_t k = 0; k < K; ++k)
            w[static_cast<std::size_t>(k)] = static_cast<float>(code_at(values + n * row_bytes, bits, k)) * scales[n * B + k / group];
        for (std::int64_t m = 0; m < M; ++m) {
            float v = 0.F;
            for (std::int64_t k = 0; k < K; ++k) v = std::fma(xr[static_cast<std::size_t>(m * K + k)], w[static_cast<std::size_t>(k)], v);
            y[m * N + n] = clampf(std::nearbyint(v / output_scale), -128.F, 127.F) * output_scale;
        }
    }
    return 0;
}

// x and residual are F32 or BF16 [rows, width] (residual may be NULL: RMS_NORM); weight F32 [width]; scale NULL or
// one float (the residual form's scalar). y F32 [rows, width]. inverse (optional) receives 1 / rms per row.
// Returns -1 for INVALID_ARGUMENT (epsilon not finite or <= 0, context.cpp:1108).
int kqr_rms_norm(const void* x, int x_dtype, std::int64_t rows, std::int64_t width, const float* weight,
                 const void* residual, const float* scale, float epsilon, float* y, float* inverse) {
    if ((x_dtype != F32 && x_dtype != BF16) || rows < 0 || width <= 0 || !std::isfinite(epsilon) || epsilon <= 0)
        return -1;
    std::vector<float> row(static_cast<std::size_t>(width));
    for (std::int64_t r = 0; r < rows; ++r) {
        for (std::int64_t i = 0; i < width; ++i) row[static_cast<std::size_t>(i)] = load_float(x, x_dtype, static_cast<std::size_t>(r * width + i));
        const float sum = rms_sum_squares(row.data(), width);
        const float inv = 1.F / std::sqrt(sum / static_cast<float>(width) + epsilon);
        if (inverse) inverse[r] = inv;
        for (std::int64_t i = 0; i < width; ++i) {
            const float n = row[static_cast<std::size_t>(i)] * inv * weight[i];
            if (!residual) {
                y[r * width + i] = n;
                continue;
            }
            const float v = load_float(residual, x_dtype, static_cast<std::size_t>(r * width + i)) + n;
            y[r * width + i] = scale ? v * scale[0] : v;
        }
    }
    return 0;
}

}  // extern "C"
