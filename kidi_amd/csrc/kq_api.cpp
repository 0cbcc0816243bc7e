// C ABI of the quantized linear layer (include/kq.h): validation, operator selection, load-time packing and
// kernel dispatch. Mirrors Kidi's contract for PACKED_LINEAR: Context::Impl::run validation
// (src/kidi/ops/context.cpp:207-218), Context::packed_linear scale checks (:821-825), the CPU backend's operator
// selection (runtime/ynn/operators.cpp:2739-2900) and its errors (core/error.h:8-14). No function throws.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/kq.h"
#include "kq_internal.hpp"

namespace {

thread_local std::string g_error;

kq_status fail(kq_status code, const std::string& message) {
    g_error = message;
    return code;
}

kq_status hip_fail(hipError_t e, const char* what) {
    return fail(KQ_RUNTIME, std::string(what) + ": " + hipGetErrorString(e));
}

float half_bits_to_float(std::uint16_t h) {
    // exact binary16 -> binary32 via the hardware-independent definition
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const std::uint32_t exponent = (h >> 10) & 0x1fu;
    std::uint32_t mantissa = h & 0x3ffu;
    std::uint32_t bits;
    if (exponent == 0x1fu) bits = sign | 0x7f800000u | (mantissa << 13);
    else if (exponent != 0) bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    else if (mantissa == 0) bits = sign;
    else {
        int shift = 0;
        while ((mantissa & 0x400u) == 0) {
            mantissa <<= 1;
            ++shift;
        }
        bits = sign | (static_cast<std::uint32_t>(113 - shift) << 23) | ((mantissa & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, sizeof f);
    return f;
}

std::size_t dtype_size(kq_dtype t) {
    switch (t) {
    case KQ_F32: return 4;
    case KQ_F16:
    case KQ_BF16: return 2;
    case KQ_U8:
    case KQ_I8:
    case KQ_ZP_U8: return 1;
    default: return 0;
    }
}

int select_path(int bits, std::int64_t group, std::int64_t K, std::int64_t N, bool has_zero, float input_scale) {
    if (input_scale <= 0.F) {
        bool blockwise = group >= 32 && K % group == 0;
        if (blockwise && bits == 4) blockwise = group % 32 == 0 && (has_zero || (group < K && N >= 256));
        else if (blockwise && bits == 8) blockwise = group % 16 == 0 && !has_zero && N >= 64;
        else blockwise = false;
        if (blockwise) return kq::PATH_BLOCKWISE;
    } else if (!has_zero && group > 0 && K % group == 0 && group % (8 / bits) == 0) {
        return kq::PATH_SYMMETRIC;
    }
    return kq::PATH_PORTABLE;
}

std::int64_t act_rows(const kq::Weight& w, std::int64_t M) {
    if (!w.tiled) return M;
    if (M <= 4) return M;
    if (M <= 8) return 8;
    return kq::round_up(M, 256);
}

constexpr std::size_t kAlign = 256;
std::size_t align_up(std::size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Grow-only scratch used when the caller passes no workspace, one per (device, stream): calls on one stream are
// ordered, so reusing that stream's buffer needs no synchronization, and calls on different streams never share
// one. Growing allocates a larger buffer and keeps the old one until the process ends (queued work may still read
// it), so no call waits for the device; growth is refused while the stream is being captured into a graph.
struct Scratch {
    void* ptr = nullptr;
    std::size_t bytes = 0;
};
std::mutex g_scratch_mutex;
using ScratchPool = std::map<std::pair<int, hipStream_t>, Scratch>;
ScratchPool g_scratch;
ScratchPool g_ffn_scratch;
ScratchPool g_greedy_scratch;
ScratchPool g_norm_scratch;
ScratchPool g_pack_scratch;
ScratchPool g_debug_scratch;  // parity instrumentation's own buffers
std::vector<void*> g_retired;  // outgrown scratch buffers, never freed while work may still be queued on them

kq_status device_scratch(ScratchPool& pool, std::size_t bytes, hipStream_t stream, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    Scratch& s = pool[{dev, stream}];
    if (s.bytes < bytes) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &capture);
        if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
        if (capture != hipStreamCaptureStatusNone)
            return fail(KQ_RUNTIME, "the library's workspace cannot grow during stream capture: pass a workspace");
        void* p = nullptr;
        e = hipMalloc(&p, std::max(bytes, s.bytes * 2));
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
        if (s.ptr) g_retired.push_back(s.ptr);
        s.ptr = p;
        s.bytes = std::max(bytes, s.bytes * 2);
    }
    *out = s.ptr;
    return KQ_OK;
}

kq_status validate_desc(const kq_pack_desc* d) {
    if (!d) return fail(KQ_INVALID_ARGUMENT, "null pack descriptor");
    const int bits = d->bits;
    if ((bits != 2 && bits != 4 && bits != 8) || d->group_size <= 0)
        return fail(KQ_INVALID_ARGUMENT, "invalid packed linear precision or group");
    if (d->rows <= 0 || d->cols <= 0 || d->cols % d->group_size || d->group_size % (8 / bits))
        return fail(KQ_INVALID_ARGUMENT, "packed linear shape or dtype mismatch");
    if (!d->values || !(d->values_dtype == KQ_U8 || (bits == 8 && d->values_dtype == KQ_I8)))
        return fail(KQ_INVALID_ARGUMENT, "packed linear shape or dtype mismatch");
    if (!d->scales || (d->scales_dtype != KQ_F32 && d->scales_dtype != KQ_F16))
        return fail(KQ_INVALID_ARGUMENT, "packed linear shape or dtype mismatch");
    if (d->zeros && d->zeros_dtype != KQ_F32 && d->zeros_dtype != KQ_F16 && d->zeros_dtype != KQ_ZP_U8)
        return fail(KQ_INVALID_ARGUMENT, "packed linear zero dtype must be F32, F16 or ZP_U8");
    if (d->memory != KQ_HOST && d->memory != KQ_DEVICE) return fail(KQ_INVALID_ARGUMENT, "invalid memory kind");
    return KQ_OK;
}

// Load-time calls (packing, import, export, weight quantization) synchronize their stream and allocate, so they
// refuse a stream that is being captured into a graph.
kq_status refuse_capture(hipStream_t stream, const char* what) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipError_t e = hipStreamIsCapturing(stream, &capture); e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (capture != hipStreamCaptureStatusNone) return fail(KQ_RUNTIME, std::string(what) + " cannot run under stream capture");
    return KQ_OK;
}

// Copy a descriptor's buffer to host memory. Device sources are read in `stream` order, after the work that
// produced them on that stream.
kq_status fetch(const void* src, std::size_t bytes, kq_memory memory, hipStream_t stream, std::vector<std::uint8_t>& out) {
    out.resize(bytes);
    if (memory == KQ_HOST) {
        std::memcpy(out.data(), src, bytes);
        return KQ_OK;
    }
    hipError_t e = hipMemcpyAsync(out.data(), src, bytes, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return hip_fail(e, "copy of a weight source");
    return KQ_OK;
}

// Offsets of the sub-buffers in a packed weight's one device allocation (-1 when absent) and its size. Both packing
// and kq_weight_import derive the image from the weight's geometry and modes with this function, so an imported
// blob is accepted only when its header describes exactly the image this library would have built.
struct ImageLayout {
    std::int64_t tiles = 0, scales = 0, zero_points = -1, zeros = -1, code_sums = -1;
    std::size_t bytes = 0;
};
ImageLayout image_layout(const kq::Weight& w) {
    const kq::Geometry& g = w.geo;
    const std::int64_t N = g.rows, B = g.cols / g.group, row_bytes = g.cols / (8 / g.bits);
    const std::size_t ssz = w.scale_type == kq::META_F16 ? 2 : 4;
    const std::size_t zsz = w.zero_type == kq::META_F16 ? 2 : 4;
    ImageLayout l;
    std::size_t off = 0;
    l.tiles = 0;
    off = align_up(off + static_cast<std::size_t>(w.tiled ? g.tile_bytes_total() : N * row_bytes));
    const std::int64_t meta_n = w.tiled ? g.meta_count() : N * B;
    l.scales = static_cast<std::int64_t>(off);
    off = align_up(off + static_cast<std::size_t>(meta_n) * ssz);
    if (w.zero_mode == kq::ZERO_POINT) {
        l.zero_points = static_cast<std::int64_t>(off);
        off = align_up(off + static_cast<std::size_t>(w.tiled ? meta_n / 2 : meta_n));
    }
    if (w.zero_mode == kq::ZERO_FLOAT) {
        l.zeros = static_cast<std::int64_t>(off);
        off = align_up(off + static_cast<std::size_t>(meta_n) * zsz);
    }
    if (w.tiled && g.bits == 8) {
        l.code_sums = static_cast<std::int64_t>(off);
        off = align_up(off + static_cast<std::size_t>(meta_n) * 4);
    }
    l.bytes = off;
    return l;
}

// Prefill copy of a 4-bit g = 128 weight for kq_gemm8.hip (layout in kq_internal.hpp): codes[N][K] signed, zp[N][K/g]
// uint4 zero points (ZERO_POINT) or null, zeros[N][K/g] additive zeros (ZERO_FLOAT) or null. Column k of a 32-column
// chunk sits at lane half (k >> 3) & 1, byte (k & 7) + 8 (k >> 4) of the column's 16-byte lane slot.
std::vector<std::uint8_t> build_prefill(const kq::Weight& w, const std::int8_t* codes, const float* scales,
                                        const std::uint8_t* zp, const float* zeros, std::size_t* codes_bytes) {
    const std::int64_t N = w.geo.rows, K = w.geo.cols, B = K / w.geo.group, NB = (N + 31) / 32, KC = K / 32;
    *codes_bytes = align_up(static_cast<std::size_t>(NB * KC) * 1024);
    std::vector<std::uint8_t> out(*codes_bytes + static_cast<std::size_t>(B * NB * 32) * 16, 0);
    for (std::int64_t n = 0; n < N; ++n) {
        const std::int64_t nb = n / 32, c = n % 32;
        for (std::int64_t k = 0; k < K; ++k) {
            const int kk = static_cast<int>(k % 32);
            const std::int64_t lane = c + 32 * ((kk >> 3) & 1), p = (kk & 7) + 8 * (kk >> 4);
            int v = codes[n * K + k];
            if (zp) v += 8 - zp[n * B + k / w.geo.group];
            out[static_cast<std::size_t>(((nb * KC + k / 32) * 64 + lane) * 16 + p)] = static_cast<std::uint8_t>(static_cast<std::int8_t>(v));
        }
        for (std::int64_t b = 0; b < B; ++b) {
            const float rec[4] = {scales[n * B + b], -12582912.F * scales[n * B + b], zeros ? zeros[n * B + b] : 0.F, 0.F};
            std::memcpy(out.data() + *codes_bytes + static_cast<std::size_t>(((b * NB + nb) * 32 + c) * 16), rec, 16);
        }
    }
    return out;
}

// Uploads a prefill copy into its own allocation (synchronous on `stream`).
kq_status upload_prefill(kq::Weight& w, const std::vector<std::uint8_t>& img, std::size_t codes_bytes, hipStream_t stream) {
    hipError_t e = hipMalloc(&w.prefill_alloc, img.size());
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(prefill copy)");
    e = hipMemcpyAsync(w.prefill_alloc, img.data(), img.size(), hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
        (void)hipFree(w.prefill_alloc);
        w.prefill_alloc = nullptr;
        return hip_fail(e, "upload prefill copy");
    }
    w.prefill_bytes = img.size();
    w.has_prefill = true;
    w.prefill_codes = static_cast<std::int8_t*>(w.prefill_alloc);
    w.prefill_meta = reinterpret_cast<float*>(static_cast<std::uint8_t*>(w.prefill_alloc) + codes_bytes);
    return KQ_OK;
}

struct HostWeight {
    std::vector<std::uint8_t> values;  // Kidi layout, all descriptors concatenated by rows
    std::vector<std::uint8_t> scales;  // [N][B] of the scale dtype
    std::vector<std::uint8_t> zeros;   // [N][B] zero dtype, empty if none
};

kq_status pack_impl(const kq_pack_desc* descs, int count, void* stream, kq_weight** out) {
    if (!out) return fail(KQ_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (!descs || count <= 0) return fail(KQ_INVALID_ARGUMENT, "no weights to pack");
    for (int i = 0; i < count; ++i)
        if (kq_status s = validate_desc(&descs[i]); s != KQ_OK) return s;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    for (int i = 0; i < count; ++i)  // device sources are read on `stream`: it must not be capturing
        if (descs[i].memory == KQ_DEVICE)
            if (kq_status s = refuse_capture(st, "packing a weight"); s != KQ_OK) return s;
    const kq_pack_desc& d0 = descs[0];
    std::int64_t N = 0;
    for (int i = 0; i < count; ++i) {
        const kq_pack_desc& d = descs[i];
        if (d.bits != d0.bits || d.group_size != d0.group_size || d.cols != d0.cols || d.scales_dtype != d0.scales_dtype ||
            (d.zeros == nullptr) != (d0.zeros == nullptr) || (d.zeros && d.zeros_dtype != d0.zeros_dtype))
            return fail(KQ_INVALID_ARGUMENT, "concatenated weights must share bits, group, K and metadata types");
        N += d.rows;
    }
    const int bits = d0.bits;
    const int group = d0.group_size;
    const std::int64_t K = d0.cols;
    const std::int64_t B = K / group;
    const std::int64_t row_bytes = K / (8 / bits);
    const std::size_t ssz = dtype_size(d0.scales_dtype);
    const bool has_zero = d0.zeros != nullptr;
    const std::size_t zsz = has_zero ? dtype_size(d0.zeros_dtype) : 0;

    HostWeight hw;
    hw.values.resize(static_cast<std::size_t>(N * row_bytes));
    hw.scales.resize(static_cast<std::size_t>(N * B) * ssz);
    if (has_zero) hw.zeros.resize(static_cast<std::size_t>(N * B) * zsz);
    std::int64_t r0 = 0;
    for (int i = 0; i < count; ++i) {
        const kq_pack_desc& d = descs[i];
        std::vector<std::uint8_t> tmp;
        if (kq_status s = fetch(d.values, static_cast<std::size_t>(d.rows * row_bytes), d.memory, st, tmp); s != KQ_OK) return s;
        std::memcpy(hw.values.data() + r0 * row_bytes, tmp.data(), tmp.size());
        if (kq_status s = fetch(d.scales, static_cast<std::size_t>(d.rows * B) * ssz, d.memory, st, tmp); s != KQ_OK) return s;
        std::memcpy(hw.scales.data() + static_cast<std::size_t>(r0 * B) * ssz, tmp.data(), tmp.size());
        if (has_zero) {
            if (kq_status s = fetch(d.zeros, static_cast<std::size_t>(d.rows * B) * zsz, d.memory, st, tmp); s != KQ_OK) return s;
            std::memcpy(hw.zeros.data() + static_cast<std::size_t>(r0 * B) * zsz, tmp.data(), tmp.size());
        }
        r0 += d.rows;
    }

    auto scale_at = [&](std::int64_t i) {
        if (d0.scales_dtype == KQ_F32) {
            float f;
            std::memcpy(&f, hw.scales.data() + 4 * i, 4);
            return f;
        }
        std::uint16_t h;
        std::memcpy(&h, hw.scales.data() + 2 * i, 2);
        return half_bits_to_float(h);
    };
    auto zero_at = [&](std::int64_t i) {
        if (d0.zeros_dtype == KQ_F32) {
            float f;
            std::memcpy(&f, hw.zeros.data() + 4 * i, 4);
            return f;
        }
        std::uint16_t h;
        std::memcpy(&h, hw.zeros.data() + 2 * i, 2);
        return half_bits_to_float(h);
    };

    auto* w = new (std::nothrow) kq::Weight();
    if (!w) return fail(KQ_RUNTIME, "out of host memory");
    w->scales_positive = true;
    for (std::int64_t i = 0; i < N * B && w->scales_positive; ++i) {
        const float sv = scale_at(i);
        w->scales_positive = std::isfinite(sv) && sv > 0.F;
    }
    w->geo = kq::Geometry::make(bits, group, N, K);
    w->tiled = kq::tiled_group_ok(bits, group);
    w->scale_type = d0.scales_dtype == KQ_F16 ? kq::META_F16 : kq::META_F32;
    w->zero_mode = kq::ZERO_NONE;
    std::vector<std::uint8_t> zp(static_cast<std::size_t>(N * B), 8);
    if (has_zero) {
        if (d0.zeros_dtype == KQ_ZP_U8) {
            for (std::int64_t i = 0; i < N * B; ++i) {
                if (hw.zeros[static_cast<std::size_t>(i)] > 15) {
                    delete w;
                    return fail(KQ_INVALID_ARGUMENT, "zero points must be in [0, 15]");
                }
                zp[static_cast<std::size_t>(i)] = hw.zeros[static_cast<std::size_t>(i)];
            }
            w->zero_mode = kq::ZERO_POINT;
        } else {
            // An additive zero of the form (8 - zp) * scale (ops::pack_weight, quantization.cpp:85) is carried as a
            // 4-bit zero point and folded into the integer partial; anything else stays a float zero.
            bool exact = bits == 4;
            for (std::int64_t i = 0; exact && i < N * B; ++i) {
                const float s = scale_at(i), z = zero_at(i);
                if (!(s != 0.F) || !std::isfinite(s) || !std::isfinite(z)) {
                    exact = false;
                    break;
                }
                const float r = 8.0F - z / s;
                const float zr = std::nearbyint(r);
                if (zr < 0.F || zr > 15.F || (8.0F - zr) * s != z) {
                    exact = false;
                    break;
                }
                zp[static_cast<std::size_t>(i)] = static_cast<std::uint8_t>(zr);
            }
            if (exact) {
                w->zero_mode = kq::ZERO_POINT;
            } else {
                w->zero_mode = kq::ZERO_FLOAT;
                w->zero_type = d0.zeros_dtype == KQ_F16 ? kq::META_F16 : kq::META_F32;
            }
        }
    }

    const kq::Geometry& g = w->geo;
    const ImageLayout lay = image_layout(*w);
    const std::size_t tiles_off = static_cast<std::size_t>(lay.tiles), scales_off = static_cast<std::size_t>(lay.scales);
    const std::size_t zp_off = static_cast<std::size_t>(std::max<std::int64_t>(lay.zero_points, 0));
    const std::size_t zeros_off = static_cast<std::size_t>(std::max<std::int64_t>(lay.zeros, 0));
    const std::size_t cs_off = static_cast<std::size_t>(std::max<std::int64_t>(lay.code_sums, 0));
    const std::size_t off = lay.bytes;
    std::vector<std::uint8_t> image(off, 0);
    if (w->tiled) {
        kq::encode_tiles(bits, N, K, hw.values.data(), image.data() + tiles_off);
        for (std::int64_t n = 0; n < N; ++n)
            for (std::int64_t b = 0; b < B; ++b) {
                const std::int64_t mi = g.meta_index(n, b), si = n * B + b;
                std::memcpy(image.data() + scales_off + static_cast<std::size_t>(mi) * ssz,
                            hw.scales.data() + static_cast<std::size_t>(si) * ssz, ssz);
                if (w->zero_mode == kq::ZERO_POINT) {
                    std::uint8_t& byte = image[zp_off + static_cast<std::size_t>((mi - n % kq::kTileRows) / 2 + (n % kq::kTileRows) / 2)];
                    byte = static_cast<std::uint8_t>(byte | (zp[static_cast<std::size_t>(si)] << (4 * (n & 1))));
                }
                if (w->zero_mode == kq::ZERO_FLOAT)
                    std::memcpy(image.data() + zeros_off + static_cast<std::size_t>(mi) * zsz,
                                hw.zeros.data() + static_cast<std::size_t>(si) * zsz, zsz);
                if (bits == 8) {
                    std::int32_t sum = 0;
                    for (std::int64_t c = 0; c < group; ++c)
                        sum += static_cast<std::int8_t>(hw.values[static_cast<std::size_t>(n * row_bytes + b * group + c)]);
                    std::memcpy(image.data() + cs_off + static_cast<std::size_t>(mi) * 4, &sum, 4);
                }
            }
    } else {
        std::memcpy(image.data() + tiles_off, hw.values.data(), hw.values.size());
        std::memcpy(image.data() + scales_off, hw.scales.data(), hw.scales.size());
        if (w->zero_mode == kq::ZERO_POINT) std::memcpy(image.data() + zp_off, zp.data(), zp.size());
        if (w->zero_mode == kq::ZERO_FLOAT) std::memcpy(image.data() + zeros_off, hw.zeros.data(), hw.zeros.size());
    }

    if (kq_status s = refuse_capture(st, "packing a weight"); s != KQ_OK) {
        delete w;
        return s;
    }
    hipError_t e = hipGetDevice(&w->device);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(e, "hipGetDevice");
    }
    e = hipMalloc(&w->allocation, off);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(e, "hipMalloc(weight)");
    }
    auto* base = static_cast<std::uint8_t*>(w->allocation);
    e = hipMemcpyAsync(base, image.data(), off, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        (void)hipFree(w->allocation);
        delete w;
        return hip_fail(e, "upload weight");
    }
    w->bytes = off;
    w->tiles = base + tiles_off;
    w->scales = base + scales_off;
    if (w->zero_mode == kq::ZERO_POINT) w->zero_points = base + zp_off;
    if (w->zero_mode == kq::ZERO_FLOAT) w->zeros = base + zeros_off;
    if (w->tiled && bits == 8) w->code_sums = reinterpret_cast<std::int32_t*>(base + cs_off);
    if (kq::gemm8_eligible(*w)) {
        std::vector<std::int8_t> codes(static_cast<std::size_t>(N * K));
        std::vector<float> sc(static_cast<std::size_t>(N * B)), zf;
        for (std::int64_t n = 0; n < N; ++n)
            for (std::int64_t k = 0; k < K; ++k)
                codes[static_cast<std::size_t>(n * K + k)] = static_cast<std::int8_t>(kq::kidi_code(hw.values.data() + n * row_bytes, bits, k));
        for (std::int64_t i = 0; i < N * B; ++i) sc[static_cast<std::size_t>(i)] = scale_at(i);
        if (w->zero_mode == kq::ZERO_FLOAT) {
            zf.resize(static_cast<std::size_t>(N * B));
            for (std::int64_t i = 0; i < N * B; ++i) zf[static_cast<std::size_t>(i)] = zero_at(i);
        }
        std::size_t cb = 0;
        const auto img = build_prefill(*w, codes.data(), sc.data(), w->zero_mode == kq::ZERO_POINT ? zp.data() : nullptr,
                                       zf.empty() ? nullptr : zf.data(), &cb);
        if (kq_status s = upload_prefill(*w, img, cb, st); s != KQ_OK) {
            (void)hipFree(w->allocation);
            delete w;
            return s;
        }
    }
    *out = reinterpret_cast<kq_weight*>(w);
    return KQ_OK;
}

const kq::Weight* as_weight(const kq_weight* w) { return reinterpret_cast<const kq::Weight*>(w); }

kq_status prepare_call(const kq_weight* weight, const kq_linear_args* args, bool gelu, kq::LinearCall& c,
                       std::size_t* ws_needed) {
    if (!weight || !args) return fail(KQ_INVALID_ARGUMENT, "null weight or arguments");
    const kq::Weight& w = *as_weight(weight);
    if (!std::isfinite(args->input_scale) || args->input_scale < 0 || !std::isfinite(args->output_scale) ||
        args->output_scale < 0)
        return fail(KQ_INVALID_ARGUMENT, "invalid calibrated projection scales");
    if (args->m < 0) return fail(KQ_INVALID_ARGUMENT, "negative row count");
    if (args->x_dtype != KQ_F32 && args->x_dtype != KQ_BF16)
        return fail(KQ_INVALID_ARGUMENT, "packed linear input must be F32 or BF16");
    if (args->m > 0 && (!args->x || !args->y)) return fail(KQ_INVALID_ARGUMENT, "null input or output");
    if (gelu && (w.geo.rows % 2)) return fail(KQ_INVALID_ARGUMENT, "GELU gate requires an even number of rows");
    c = kq::LinearCall{};
    c.w = &w;
    c.x = args->x;
    c.x_type = args->x_dtype == KQ_BF16 ? kq::ACT_BF16 : kq::ACT_F32;
    c.M = args->m;
    c.input_scale = args->input_scale;
    c.output_scale = args->output_scale;
    c.y = args->y;
    c.path = select_path(w.geo.bits, w.geo.group, w.geo.cols, w.geo.rows, w.zero_mode != kq::ZERO_NONE, args->input_scale);
    c.gelu_gate = gelu;
    *ws_needed = c.path == kq::PATH_PORTABLE ? 0 : kq::workspace_bytes(w, c.M);
    return KQ_OK;
}

// The kernel sequence of a prepared call. Workspace-independent: the predicates read shapes, modes and (for the g = 32
// / 64 GEMM's 16-byte loads) the input's alignment only.
kq::Route route_of(const kq::LinearCall& c, kq::SkinnyPlan* plan) {
    if (c.M == 0) return kq::ROUTE_NONE;
    if (kq::decode_fits(c)) return kq::ROUTE_DECODE;
    kq::SkinnyPlan p;
    if (kq::skinny_plan(c, p)) {
        if (plan) *plan = p;
        return kq::ROUTE_SKINNY;
    }
    if (kq::gemm8_fits(c)) return kq::gemm8_plan(*c.w, c.M, c.gelu_gate).wide && !c.dump ? kq::ROUTE_GEMM8W : kq::ROUTE_GEMM8;
    if (kq::gemm_i4_fits(c)) return kq::ROUTE_GEMM_I4;
    if (kq::gemm_i4g_fits(c)) return kq::ROUTE_GEMM_I4G;
    if (c.path == kq::PATH_PORTABLE) return kq::ROUTE_PORTABLE;
    if (!c.w->tiled) return kq::ROUTE_ROWMAJOR;
    return c.M <= 8 ? kq::ROUTE_GEMV : kq::ROUTE_GEMM;
}

kq_status run_call(kq::LinearCall& c, const kq_linear_args* args, std::size_t ws_needed, hipStream_t stream) {
    if (c.M == 0) return KQ_OK;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev != c.w->device) return fail(KQ_INVALID_ARGUMENT, "weight was packed on another device");
    kq::SkinnyPlan plan;
    const kq::Route route = route_of(c, &plan);
    // Decode shapes: one fused launch, no workspace.
    if (route == kq::ROUTE_DECODE) {
        e = kq::launch_decode(c, stream);
        return e == hipSuccess ? KQ_OK : hip_fail(e, "decode projection launch");
    }
    if (route == kq::ROUTE_SKINNY) {
        e = kq::launch_skinny(c, plan, stream);
        return e == hipSuccess ? KQ_OK : hip_fail(e, "skinny projection launch");
    }
    void* ws = args->workspace;
    if (ws_needed) {
        if (ws) {
            if (args->workspace_bytes < ws_needed) return fail(KQ_INVALID_ARGUMENT, "workspace too small");
        } else if (kq_status s = device_scratch(g_scratch, ws_needed, stream, &ws); s != KQ_OK) {
            return s;
        }
        c.act = kq::carve_workspace(*c.w, c.M, ws);
    }
    // Prefill, 4-bit g = 128 from the weight's prefill copy: quantizer + int8 GEMM (GELU gate fused).
    if (route == kq::ROUTE_GEMM8 || route == kq::ROUTE_GEMM8W) {
        e = kq::launch_gemm8(c, c.act, stream);
        return e == hipSuccess ? KQ_OK : hip_fail(e, "prefill projection launch");
    }
    // Prefill, 4-bit g = 128: quantizer + int8 MFMA GEMM (GELU gate fused).
    if (route == kq::ROUTE_GEMM_I4) {
        e = kq::launch_gemm_i4(c, c.act, stream);
        return e == hipSuccess ? KQ_OK : hip_fail(e, "prefill projection launch");
    }
    // Prefill, 4-bit g = 32 / 64 (fused QKV): quantizer + two-stage int8 MFMA GEMM.
    if (route == kq::ROUTE_GEMM_I4G) {
        e = kq::launch_gemm_i4g(c, stream);
        return e == hipSuccess ? KQ_OK : hip_fail(e, "prefill projection launch");
    }
    // GELU gating is fused everywhere except in the tiled GEMV/GEMM when the gate/up split falls inside a 16-row
    // tile: the full projection then goes to the workspace's temp and a gating kernel follows.
    float* final_y = c.y;
    if (c.gelu_gate && (route == kq::ROUTE_GEMV || route == kq::ROUTE_GEMM) && kq::gelu_needs_temp(*c.w)) {
        c.y = c.act.gelu_tmp;
        c.gelu_gate = false;
    }
    e = kq::launch_quantize(c, stream);
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
    e = kq::launch_linear(c, stream);
    if (e != hipSuccess) return hip_fail(e, "projection launch");
    if (c.y != final_y) {
        e = kq::launch_gelu_gate(c.y, c.M, c.w->geo.rows / 2, final_y, stream);
        if (e != hipSuccess) return hip_fail(e, "gelu gate launch");
    }
    return KQ_OK;
}

// Gated feed-forward workspace: h [M, I], the full gate/up projection [M, 2I] (SiLU gating runs as its own pass),
// then the larger of the two projections' workspaces (they run one after the other on the stream).
struct FfnLayout {
    std::size_t h = 0, full = 0, proj = 0;
    std::size_t total() const { return h + full + proj; }
};
FfnLayout ffn_layout(const kq::Weight& gu, const kq::Weight& dn, std::int64_t M) {
    FfnLayout l;
    const std::int64_t I = gu.geo.rows / 2;
    l.h = align_up(static_cast<std::size_t>(M * I) * 4);
    l.full = align_up(static_cast<std::size_t>(M * gu.geo.rows) * 4);
    l.proj = std::max(kq::workspace_bytes(gu, M), kq::workspace_bytes(dn, M));
    return l;
}

kq_status ffn_validate(const kq_weight* gate_up, const kq_weight* down, const kq_ffn_args* a) {
    if (!gate_up || !down || !a) return fail(KQ_INVALID_ARGUMENT, "null weight or arguments");
    const kq::Weight& gu = *as_weight(gate_up);
    const kq::Weight& dn = *as_weight(down);
    if (gu.geo.rows % 2 || dn.geo.cols != gu.geo.rows / 2 || dn.geo.rows != gu.geo.cols || dn.geo.bits != gu.geo.bits)
        return fail(KQ_INVALID_ARGUMENT, "gated feed-forward weights must be gate_up [2I, K] and down [K, I] of equal bits");
    for (float v : {a->gate_up_input_scale, a->gate_up_output_scale, a->down_input_scale, a->down_output_scale})
        if (!std::isfinite(v) || v < 0) return fail(KQ_INVALID_ARGUMENT, "invalid calibrated projection scales");
    if (a->m < 0) return fail(KQ_INVALID_ARGUMENT, "negative row count");
    if (a->x_dtype != KQ_F32 && a->x_dtype != KQ_BF16) return fail(KQ_INVALID_ARGUMENT, "feed-forward input must be F32 or BF16");
    if (a->m > 0 && (!a->x || !a->y)) return fail(KQ_INVALID_ARGUMENT, "null input or output");
    if (gu.device != dn.device) return fail(KQ_INVALID_ARGUMENT, "weights were packed on different devices");
    return KQ_OK;
}

// Persisted layout blob: this header, then the weight's device image (one allocation; sub-buffers at offsets).
constexpr char kBlobMagic[8] = {'K', 'Q', 'G', 'F', 'X', '9', '5', '0'};
constexpr std::uint32_t kBlobVersion = 1;  // bump with any change to the tile layout or this header
struct BlobHeader {
    char magic[8];
    std::uint32_t version;
    std::int32_t bits, group;
    std::int64_t rows, cols;
    std::int32_t tiled, scale_type, zero_mode, zero_type;
    std::int64_t tiles, scales, zero_points, zeros, code_sums;  // byte offsets in the image, -1 when absent
    std::uint64_t bytes;                                         // image size
};

// Greedy-head workspace: the projection's workspace, logits [M, N] (when the caller keeps none), and the selection
// partials (at most one per row tile and row: decode workgroups and 4096-column chunks are both fewer).
struct GreedyLayout {
    std::size_t lin = 0, logits = 0, parts = 0;
    std::size_t total() const { return lin + logits + parts; }
};
GreedyLayout greedy_layout(const kq::Weight& w, std::int64_t M) {
    GreedyLayout l;
    l.lin = align_up(kq::workspace_bytes(w, M));
    l.logits = align_up(static_cast<std::size_t>(M * w.geo.rows) * 4);
    const std::int64_t parts = std::max<std::int64_t>(w.geo.n_tiles, kq::greedy_chunk_count(w.geo.rows));
    l.parts = align_up(static_cast<std::size_t>(M * parts) * 16);
    return l;
}

// Normalized-projection workspace: the projection's own workspace, the normalized input [M, K] F32 (paths without a
// fused normalization), the per-row inverse RMS [M] (prefill quantizer).
struct RmsLayout {
    std::size_t lin = 0, norm = 0, inv = 0;
    std::size_t total() const { return lin + norm + inv; }
};
RmsLayout rms_layout(const kq::Weight& w, std::int64_t M) {
    RmsLayout l;
    l.lin = align_up(kq::workspace_bytes(w, M));
    l.norm = align_up(static_cast<std::size_t>(M * w.geo.cols) * 4);
    l.inv = align_up(static_cast<std::size_t>(M) * 4);
    return l;
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// Context::rms_norm / rms_norm_residual operand checks (ops/context.cpp:1103-1112): epsilon finite and > 0.
kq_status norm_validate(const kq_norm_desc* n) {
    if (!n || !n->weight) return fail(KQ_INVALID_ARGUMENT, "invalid RMS residual normalization operands");
    if (!std::isfinite(n->epsilon) || n->epsilon <= 0) return fail(KQ_INVALID_ARGUMENT, "invalid RMS residual normalization operands");
    if (n->residual && (!n->residual_weight || !n->hidden || !std::isfinite(n->residual_epsilon) || n->residual_epsilon <= 0))
        return fail(KQ_INVALID_ARGUMENT, "invalid RMS residual normalization operands");
    return KQ_OK;
}

}  // namespace

namespace kq {

namespace {
// Partial tiles of a K-split prefill GEMM (kq_gemm.hip): the larger of the plans with and without GELU gating, 0
// where that GEMM does not run or does not split.
std::size_t split_bytes(const Weight& w, std::int64_t M) {
    std::size_t partial = 0;
    if (gemm8_eligible(w) && M > 16) {
        partial = gemm8_partial_bytes(w, M, false);
        if (w.geo.rows % 64 == 0) partial = std::max(partial, gemm8_partial_bytes(w, M, true));
        partial = align_up(partial);
    }
    if (!w.tiled || w.geo.bits != 4 || w.geo.group != 128 || M <= 16 || w.geo.cols % 512 || w.geo.cols_p != w.geo.cols)
        return partial;
    for (int gelu = 0; gelu < 2; ++gelu) {
        if (gelu && ((w.geo.rows / 2) % kTileRows || w.geo.n_tiles % 2)) continue;
        const GemmPlan p = gemm_i4_plan(w, M, gelu != 0);
        if (p.ksplit == 1) continue;
        const std::size_t tiles = static_cast<std::size_t>(p.m_blocks) * p.n_blocks;
        partial = std::max(partial, align_up(static_cast<std::size_t>(p.ksplit) * tiles * (128 * p.wm) * 64 * 4));
    }
    return partial;
}
}  // namespace

int set_error(int code, const char* message) { return fail(static_cast<kq_status>(code), message); }

bool gelu_needs_temp(const Weight& w) { return w.tiled && w.geo.rows % 2 == 0 && (w.geo.rows / 2) % kTileRows != 0; }

std::size_t workspace_bytes(const Weight& w, std::int64_t M) {
    const std::int64_t rows = act_rows(w, M);
    const std::int64_t cols = w.tiled ? w.geo.cols_p : w.geo.cols;
    const std::int64_t groups = w.tiled ? w.geo.groups_p : w.geo.cols / w.geo.group;
    return align_up(static_cast<std::size_t>(rows * cols)) + 3 * align_up(static_cast<std::size_t>(rows * groups) * 4) +
           split_bytes(w, M) + (gelu_needs_temp(w) ? align_up(static_cast<std::size_t>(M * w.geo.rows) * 4) : 0);
}

ActBuffers carve_workspace(const Weight& w, std::int64_t M, void* base) {
    ActBuffers a;
    a.rows_p = act_rows(w, M);
    const std::int64_t cols = w.tiled ? w.geo.cols_p : w.geo.cols;
    const std::int64_t groups = w.tiled ? w.geo.groups_p : w.geo.cols / w.geo.group;
    auto* p = static_cast<std::uint8_t*>(base);
    a.q = reinterpret_cast<std::int8_t*>(p);
    p += align_up(static_cast<std::size_t>(a.rows_p * cols));
    a.scale = reinterpret_cast<float*>(p);
    p += align_up(static_cast<std::size_t>(a.rows_p * groups) * 4);
    a.sum = reinterpret_cast<std::int32_t*>(p);
    p += align_up(static_cast<std::size_t>(a.rows_p * groups) * 4);
    a.zero = reinterpret_cast<std::int32_t*>(p);
    p += align_up(static_cast<std::size_t>(a.rows_p * groups) * 4);
    if (const std::size_t sb = split_bytes(w, M)) {
        a.partial = reinterpret_cast<float*>(p);
        p += sb;
    }
    if (gelu_needs_temp(w)) a.gelu_tmp = reinterpret_cast<float*>(p);
    return a;
}

}  // namespace kq

extern "C" {

const char* kq_last_error(void) { return g_error.c_str(); }

int32_t kq_version(void) { return 1; }

const char* kq_arch(void) { return "gfx950"; }

kq_status kq_weight_pack(const kq_pack_desc* desc, void* stream, kq_weight** out) { return pack_impl(desc, 1, stream, out); }

kq_status kq_weight_pack_concat(const kq_pack_desc* descs, int32_t count, void* stream, kq_weight** out) {
    return pack_impl(descs, count, stream, out);
}

size_t kq_weight_export_size(const kq_weight* weight) {
    if (!weight) return 0;
    return sizeof(BlobHeader) + as_weight(weight)->bytes;
}

kq_status kq_weight_export(const kq_weight* weight, void* host, size_t bytes, void* stream) {
    if (!weight || !host) return fail(KQ_INVALID_ARGUMENT, "null weight or buffer");
    const kq::Weight& w = *as_weight(weight);
    if (bytes < sizeof(BlobHeader) + w.bytes) return fail(KQ_INVALID_ARGUMENT, "export buffer too small");
    if (kq_status s = refuse_capture(static_cast<hipStream_t>(stream), "exporting a weight"); s != KQ_OK) return s;
    BlobHeader h{};
    std::memcpy(h.magic, kBlobMagic, sizeof(h.magic));
    h.version = kBlobVersion;
    h.bits = w.geo.bits;
    h.group = w.geo.group;
    h.rows = w.geo.rows;
    h.cols = w.geo.cols;
    h.tiled = w.tiled;
    h.scale_type = w.scale_type;
    h.zero_mode = w.zero_mode;
    h.zero_type = w.zero_type;
    const auto* base = static_cast<const std::uint8_t*>(w.allocation);
    auto off = [&](const void* p) { return p ? static_cast<std::int64_t>(static_cast<const std::uint8_t*>(p) - base) : -1; };
    h.tiles = off(w.tiles);
    h.scales = off(w.scales);
    h.zero_points = off(w.zero_points);
    h.zeros = off(w.zeros);
    h.code_sums = off(w.code_sums);
    h.bytes = w.bytes;
    std::memcpy(host, &h, sizeof(h));
    auto* dst = static_cast<std::uint8_t*>(host) + sizeof(h);
    hipError_t e = hipMemcpyAsync(dst, w.allocation, w.bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "export weight");
    return KQ_OK;
}

kq_status kq_weight_import(const void* host, size_t bytes, void* stream, kq_weight** out) {
    if (!host || !out) return fail(KQ_INVALID_ARGUMENT, "null blob or output");
    *out = nullptr;
    BlobHeader h{};
    if (bytes < sizeof(h)) return fail(KQ_INVALID_MANIFEST, "packed weight blob too short");
    std::memcpy(&h, host, sizeof(h));
    if (std::memcmp(h.magic, kBlobMagic, sizeof(h.magic)) != 0 || h.version != kBlobVersion)
        return fail(KQ_INVALID_MANIFEST, "not a packed weight blob of this layout version");
    // The header must describe exactly the image pack_impl builds for its geometry and modes: the same PACKED_LINEAR
    // shape rules (context.cpp:207-218), modes in range, the tiled flag the geometry implies, and every offset and the
    // size equal to what image_layout() derives. Anything else could send a kernel past the allocation.
    const bool ok_bits = h.bits == 2 || h.bits == 4 || h.bits == 8;
    if (!ok_bits || h.group <= 0 || h.rows <= 0 || h.cols <= 0 || h.cols % h.group || h.group % (8 / h.bits) ||
        h.rows >= (std::int64_t{1} << 40) || h.cols >= (std::int64_t{1} << 32) || bytes != sizeof(h) + h.bytes ||
        h.bytes == 0)
        return fail(KQ_INVALID_MANIFEST, "malformed packed weight blob");
    if ((h.scale_type != kq::META_F32 && h.scale_type != kq::META_F16) ||
        (h.zero_mode != kq::ZERO_NONE && h.zero_mode != kq::ZERO_POINT && h.zero_mode != kq::ZERO_FLOAT) ||
        (h.zero_type != kq::META_F32 && h.zero_type != kq::META_F16) || (h.tiled != 0) != kq::tiled_group_ok(h.bits, h.group))
        return fail(KQ_INVALID_MANIFEST, "malformed packed weight blob");
    auto* w = new kq::Weight{};
    w->geo = kq::Geometry::make(h.bits, h.group, h.rows, h.cols);
    w->tiled = h.tiled != 0;
    w->scale_type = h.scale_type;
    w->zero_mode = h.zero_mode;
    w->zero_type = h.zero_type;
    const ImageLayout lay = image_layout(*w);
    if (h.tiles != lay.tiles || h.scales != lay.scales || h.zero_points != lay.zero_points || h.zeros != lay.zeros ||
        h.code_sums != lay.code_sums || h.bytes != lay.bytes) {
        delete w;
        return fail(KQ_INVALID_MANIFEST, "malformed packed weight blob");
    }
    if (kq_status s = refuse_capture(static_cast<hipStream_t>(stream), "importing a weight"); s != KQ_OK) {
        delete w;
        return s;
    }
    {
        const auto* img = static_cast<const std::uint8_t*>(host) + sizeof(h);
        const std::int64_t B = h.cols / h.group;
        w->scales_positive = true;
        for (std::int64_t n = 0; n < h.rows && w->scales_positive; ++n)
            for (std::int64_t b = 0; b < B && w->scales_positive; ++b) {
                const std::int64_t i = w->tiled ? w->geo.meta_index(n, b) : n * B + b;
                float sv;
                if (h.scale_type == kq::META_F16) {
                    std::uint16_t hb;
                    std::memcpy(&hb, img + h.scales + 2 * i, 2);
                    sv = half_bits_to_float(hb);
                } else {
                    std::memcpy(&sv, img + h.scales + 4 * i, 4);
                }
                w->scales_positive = std::isfinite(sv) && sv > 0.F;
            }
    }
    hipError_t e = hipGetDevice(&w->device);
    if (e == hipSuccess) e = hipMalloc(&w->allocation, h.bytes);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(e, "hipMalloc(weight)");
    }
    auto* base = static_cast<std::uint8_t*>(w->allocation);
    e = hipMemcpyAsync(base, static_cast<const std::uint8_t*>(host) + sizeof(h), h.bytes, hipMemcpyHostToDevice,
                       static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        (void)hipFree(w->allocation);
        delete w;
        return hip_fail(e, "import weight");
    }
    w->bytes = h.bytes;
    auto at = [&](std::int64_t o) -> std::uint8_t* { return o < 0 ? nullptr : base + o; };
    w->tiles = at(h.tiles);
    w->scales = at(h.scales);
    w->zero_points = at(h.zero_points);
    w->zeros = at(h.zeros);
    w->code_sums = reinterpret_cast<std::int32_t*>(at(h.code_sums));
    if (kq::gemm8_eligible(*w)) {  // the prefill copy is derived from the image, not stored in the blob
        const auto* img = static_cast<const std::uint8_t*>(host) + sizeof(h);
        const std::int64_t N = h.rows, K = h.cols, B = K / h.group;
        std::vector<std::int8_t> codes(static_cast<std::size_t>(N * K));
        kq::decode_tiles(h.bits, N, K, img + h.tiles, codes.data());
        std::vector<float> sc(static_cast<std::size_t>(N * B)), zf;
        std::vector<std::uint8_t> zpv;
        auto meta_float = [&](std::int64_t off, int type, std::int64_t i) {
            float f;
            if (type == kq::META_F16) {
                std::uint16_t hb;
                std::memcpy(&hb, img + off + 2 * i, 2);
                f = half_bits_to_float(hb);
            } else {
                std::memcpy(&f, img + off + 4 * i, 4);
            }
            return f;
        };
        if (h.zero_mode == kq::ZERO_POINT) zpv.resize(static_cast<std::size_t>(N * B));
        if (h.zero_mode == kq::ZERO_FLOAT) zf.resize(static_cast<std::size_t>(N * B));
        for (std::int64_t n = 0; n < N; ++n)
            for (std::int64_t b = 0; b < B; ++b) {
                const std::int64_t mi = w->geo.meta_index(n, b), i = n * B + b;
                sc[static_cast<std::size_t>(i)] = meta_float(h.scales, h.scale_type, mi);
                if (h.zero_mode == kq::ZERO_POINT)
                    zpv[static_cast<std::size_t>(i)] = static_cast<std::uint8_t>(
                        (img[h.zero_points + (mi - n % kq::kTileRows) / 2 + (n % kq::kTileRows) / 2] >> (4 * (n & 1))) & 15);
                if (h.zero_mode == kq::ZERO_FLOAT) zf[static_cast<std::size_t>(i)] = meta_float(h.zeros, h.zero_type, mi);
            }
        std::size_t cb = 0;
        const auto pimg = build_prefill(*w, codes.data(), sc.data(), zpv.empty() ? nullptr : zpv.data(),
                                        zf.empty() ? nullptr : zf.data(), &cb);
        if (kq_status s = upload_prefill(*w, pimg, cb, static_cast<hipStream_t>(stream)); s != KQ_OK) {
            (void)hipFree(w->allocation);
            delete w;
            return s;
        }
    }
    *out = reinterpret_cast<kq_weight*>(w);
    return KQ_OK;
}

void kq_weight_free(kq_weight* weight) {
    if (!weight) return;
    auto* w = reinterpret_cast<kq::Weight*>(weight);
    if (w->allocation) (void)hipFree(w->allocation);
    if (w->prefill_alloc) (void)hipFree(w->prefill_alloc);
    delete w;
}

kq_status kq_weight_info(const kq_weight* weight, int32_t* bits, int32_t* group_size, int64_t* rows, int64_t* cols,
                         int32_t* has_zeros, size_t* device_bytes) {
    if (!weight) return fail(KQ_INVALID_ARGUMENT, "null weight");
    const kq::Weight& w = *as_weight(weight);
    if (bits) *bits = w.geo.bits;
    if (group_size) *group_size = w.geo.group;
    if (rows) *rows = w.geo.rows;
    if (cols) *cols = w.geo.cols;
    if (has_zeros) *has_zeros = w.zero_mode != kq::ZERO_NONE;
    if (device_bytes) *device_bytes = w.bytes + w.prefill_bytes;
    return KQ_OK;
}

int32_t kq_select_path(int32_t bits, int64_t group_size, int64_t cols, int64_t rows, int32_t has_zeros, float input_scale) {
    if ((bits != 2 && bits != 4 && bits != 8) || group_size <= 0) return -1;
    return select_path(bits, group_size, cols, rows, has_zeros != 0, input_scale);
}

size_t kq_linear_workspace_size(const kq_weight* weight, int64_t m) {
    if (!weight || m < 0) return 0;
    return kq::workspace_bytes(*as_weight(weight), m);
}

kq_status kq_packed_linear(const kq_weight* weight, const kq_linear_args* args, void* stream) {
    kq::LinearCall c;
    std::size_t ws = 0;
    if (kq_status s = prepare_call(weight, args, false, c, &ws); s != KQ_OK) return s;
    return run_call(c, args, ws, static_cast<hipStream_t>(stream));
}

kq_status kq_packed_linear_gelu_gate(const kq_weight* weight, const kq_linear_args* args, void* stream) {
    kq::LinearCall c;
    std::size_t ws = 0;
    if (kq_status s = prepare_call(weight, args, true, c, &ws); s != KQ_OK) return s;
    return run_call(c, args, ws, static_cast<hipStream_t>(stream));
}

size_t kq_ffn_workspace_size(const kq_weight* gate_up, const kq_weight* down, int64_t m) {
    if (!gate_up || !down || m < 0) return 0;
    return ffn_layout(*as_weight(gate_up), *as_weight(down), m).total();
}

kq_status kq_gated_feed_forward(const kq_weight* gate_up, const kq_weight* down, const kq_ffn_args* args, void* stream) {
    if (kq_status s = ffn_validate(gate_up, down, args); s != KQ_OK) return s;
    if (args->m == 0) return KQ_OK;
    const kq::Weight& gu = *as_weight(gate_up);
    const kq::Weight& dn = *as_weight(down);
    const FfnLayout l = ffn_layout(gu, dn, args->m);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = args->workspace;
    if (ws) {
        if (args->workspace_bytes < l.total()) return fail(KQ_INVALID_ARGUMENT, "workspace too small");
    } else if (kq_status s = device_scratch(g_ffn_scratch, l.total(), st, &ws); s != KQ_OK) {
        return s;
    }
    auto* base = static_cast<std::uint8_t*>(ws);
    float* h = reinterpret_cast<float*>(base);
    float* full = reinterpret_cast<float*>(base + l.h);
    void* proj = base + l.h + l.full;
    kq_linear_args a{};
    a.x = args->x;
    a.x_dtype = args->x_dtype;
    a.m = args->m;
    a.input_scale = args->gate_up_input_scale;
    a.output_scale = args->gate_up_output_scale;
    a.workspace = proj;
    a.workspace_bytes = l.proj;
    if (args->silu) {
        a.y = full;
        if (kq_status s = kq_packed_linear(gate_up, &a, stream); s != KQ_OK) return s;
        if (hipError_t e = kq::launch_silu_gate(full, args->m, gu.geo.rows / 2, h, st); e != hipSuccess)
            return hip_fail(e, "SiLU gate launch");
    } else {
        a.y = h;
        if (kq_status s = kq_packed_linear_gelu_gate(gate_up, &a, stream); s != KQ_OK) return s;
    }
    a.x = h;
    a.x_dtype = KQ_F32;
    a.input_scale = args->down_input_scale;
    a.output_scale = args->down_output_scale;
    a.y = args->y;
    return kq_packed_linear(down, &a, stream);
}

size_t kq_greedy_workspace_size(int64_t rows, int64_t width) {
    if (rows < 0 || width < 1) return 0;
    return align_up(static_cast<std::size_t>(rows * kq::greedy_chunk_count(width)) * 16);
}

static kq_status gated_multiply(const float* gate, const float* value, int64_t count, float* y, bool silu, void* stream) {
    if (count < 0) return fail(KQ_INVALID_ARGUMENT, silu ? "SiLU multiplication requires matching floating tensors"
                                                         : "GELU multiplication requires matching floating tensors");
    if (count == 0) return KQ_OK;
    if (!gate || !value || !y) return fail(KQ_INVALID_ARGUMENT, "null gate, value or output");
    if (hipError_t e = kq::launch_gated_multiply(gate, value, count, silu, y, static_cast<hipStream_t>(stream)); e != hipSuccess)
        return hip_fail(e, "gated multiply launch");
    return KQ_OK;
}

kq_status kq_gelu_multiply(const float* gate, const float* value, int64_t count, float* y, void* stream) {
    return gated_multiply(gate, value, count, y, false, stream);
}

kq_status kq_silu_multiply(const float* gate, const float* value, int64_t count, float* y, void* stream) {
    return gated_multiply(gate, value, count, y, true, stream);
}

kq_status kq_greedy_token(const float* logits, int64_t rows, int64_t width, int32_t* tokens, void* workspace,
                          size_t workspace_bytes, void* stream) {
    if (rows < 0 || width < 1) return fail(KQ_INVALID_ARGUMENT, "greedy selection requires [rows, width > 0] logits");
    if (rows == 0) return KQ_OK;
    if (!logits || !tokens) return fail(KQ_INVALID_ARGUMENT, "null logits or tokens");
    const std::size_t need = kq_greedy_workspace_size(rows, width);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = workspace;
    if (ws) {
        if (workspace_bytes < need) return fail(KQ_INVALID_ARGUMENT, "workspace too small");
    } else if (kq_status s = device_scratch(g_greedy_scratch, need, st, &ws); s != KQ_OK) {
        return s;
    }
    auto* parts = static_cast<int4*>(ws);
    if (hipError_t e = kq::launch_greedy_chunks(logits, rows, width, parts, st); e != hipSuccess) return hip_fail(e, "greedy launch");
    if (hipError_t e = kq::launch_greedy_reduce(parts, rows, kq::greedy_chunk_count(width), tokens, st); e != hipSuccess)
        return hip_fail(e, "greedy launch");
    return KQ_OK;
}

size_t kq_greedy_linear_workspace_size(const kq_weight* weight, int64_t m) {
    if (!weight || m < 0) return 0;
    return greedy_layout(*as_weight(weight), m).total();
}

kq_status kq_packed_linear_greedy(const kq_weight* weight, const kq_linear_args* args, int32_t* tokens, void* stream) {
    if (!weight || !args) return fail(KQ_INVALID_ARGUMENT, "null weight or arguments");
    if (args->m > 0 && !tokens) return fail(KQ_INVALID_ARGUMENT, "null tokens");
    const kq::Weight& w = *as_weight(weight);
    const GreedyLayout l = greedy_layout(w, std::max<int64_t>(args->m, 0));
    void* ws = args->workspace;
    if (args->m > 0) {
        if (ws) {
            if (args->workspace_bytes < l.total()) return fail(KQ_INVALID_ARGUMENT, "workspace too small");
        } else if (kq_status s = device_scratch(g_greedy_scratch, l.total(), static_cast<hipStream_t>(stream), &ws); s != KQ_OK) {
            return s;
        }
    }
    auto* base = static_cast<std::uint8_t*>(ws);
    kq_linear_args la = *args;
    la.workspace = base;
    la.workspace_bytes = l.lin;
    if (!la.y && base) la.y = reinterpret_cast<float*>(base + l.lin);
    kq::LinearCall c;
    std::size_t need = 0;
    if (kq_status s = prepare_call(weight, &la, false, c, &need); s != KQ_OK) return s;
    if (c.M == 0) return KQ_OK;
    auto* parts = reinterpret_cast<int4*>(base + l.lin + l.logits);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev != w.device) return fail(KQ_INVALID_ARGUMENT, "weight was packed on another device");
    if (kq::decode_fits(c)) {
        int count = 0;
        c.y = args->y;  // NULL: the logits stay on chip
        c.greedy = parts;
        c.greedy_parts = &count;
        if (hipError_t e = kq::launch_decode(c, st); e != hipSuccess) return hip_fail(e, "decode projection launch");
        if (hipError_t e = kq::launch_greedy_reduce(parts, c.M, count, tokens, st); e != hipSuccess) return hip_fail(e, "greedy launch");
        return KQ_OK;
    }
    if (kq_status s = run_call(c, &la, need, st); s != KQ_OK) return s;
    if (hipError_t e = kq::launch_greedy_chunks(la.y, c.M, w.geo.rows, parts, st); e != hipSuccess) return hip_fail(e, "greedy launch");
    if (hipError_t e = kq::launch_greedy_reduce(parts, c.M, kq::greedy_chunk_count(w.geo.rows), tokens, st); e != hipSuccess)
        return hip_fail(e, "greedy launch");
    return KQ_OK;
}

kq_status kq_rms_norm(const kq_rms_args* args, void* stream) {
    if (!args) return fail(KQ_INVALID_ARGUMENT, "null arguments");
    if (args->rows < 0 || args->width <= 0 || (args->x_dtype != KQ_F32 && args->x_dtype != KQ_BF16) || !args->weight ||
        !std::isfinite(args->epsilon) || args->epsilon <= 0)
        return fail(KQ_INVALID_ARGUMENT, "invalid RMS residual normalization operands");
    if (args->rows == 0) return KQ_OK;
    if (!args->x || !args->y) return fail(KQ_INVALID_ARGUMENT, "null input or output");
    if (args->output_scale && !args->residual)
        return fail(KQ_INVALID_ARGUMENT, "an output scale needs the residual form");
    kq::NormLaunch n;
    n.x = args->x;
    n.x_type = args->x_dtype == KQ_BF16 ? kq::ACT_BF16 : kq::ACT_F32;
    n.residual = args->residual;
    n.w1 = args->weight;
    n.scale = args->output_scale;
    n.out1 = args->y;
    n.rows = args->rows;
    n.width = args->width;
    n.eps1 = args->epsilon;
    if (hipError_t e = kq::launch_rms_norm(n, static_cast<hipStream_t>(stream)); e != hipSuccess)
        return hip_fail(e, "RMS normalization launch");
    return KQ_OK;
}

size_t kq_rms_linear_workspace_size(const kq_weight* weight, int64_t m) {
    if (!weight || m < 0) return 0;
    return rms_layout(*as_weight(weight), m).total();
}

kq_status kq_packed_linear_rms(const kq_weight* weight, const kq_linear_args* args, const kq_norm_desc* norm,
                               int32_t gelu_gate, void* stream) {
    kq::LinearCall c;
    std::size_t ws_lin = 0;
    if (kq_status s = prepare_call(weight, args, gelu_gate != 0, c, &ws_lin); s != KQ_OK) return s;
    if (kq_status s = norm_validate(norm); s != KQ_OK) return s;
    if (c.M == 0) return KQ_OK;
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev != c.w->device) return fail(KQ_INVALID_ARGUMENT, "weight was packed on another device");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool res = norm->residual != nullptr;
    const std::int64_t K = c.w->geo.cols;
    // Decode (M <= 8, K <= 2048): the projection kernel normalizes its own input (one launch).
    c.norm = res ? 2 : 1;
    c.norm_w1 = res ? norm->residual_weight : norm->weight;
    c.norm_w2 = res ? norm->weight : nullptr;
    c.norm_res = norm->residual;
    c.norm_scale = norm->residual_scale;
    c.norm_hidden = norm->hidden;
    c.norm_eps1 = res ? norm->residual_epsilon : norm->epsilon;
    c.norm_eps2 = norm->epsilon;
    const bool aligned = aligned16(c.norm_w1) && (!res || (aligned16(norm->weight) && aligned16(norm->hidden) &&
                                                           aligned16(norm->residual)));
    if (aligned && kq::decode_fits(c)) {
        if (hipError_t e = kq::launch_decode(c, st); e != hipSuccess) return hip_fail(e, "decode projection launch");
        return KQ_OK;
    }
    c.norm = 0;
    const RmsLayout l = rms_layout(*c.w, c.M);
    void* ws = args->workspace;
    if (ws) {
        if (args->workspace_bytes < l.total()) return fail(KQ_INVALID_ARGUMENT, "workspace too small");
    } else if (kq_status s = device_scratch(g_norm_scratch, l.total(), st, &ws); s != KQ_OK) {
        return s;
    }
    auto* base = static_cast<std::uint8_t*>(ws);
    float* normed = reinterpret_cast<float*>(base + l.lin);
    float* inv = reinterpret_cast<float*>(base + l.lin + l.norm);
    kq::NormLaunch n;
    n.x = args->x;
    n.x_type = c.x_type;
    n.residual = norm->residual;
    n.w1 = c.norm_w1;
    n.scale = norm->residual_scale;
    n.rows = c.M;
    n.width = K;
    n.eps1 = c.norm_eps1;
    n.eps2 = norm->epsilon;
    // Prefill 4-bit g = 128: per-row statistics (and h), then the row quantizer normalizes while it quantizes.
    if (ws_lin) c.act = kq::carve_workspace(*c.w, c.M, base);
    kq::LinearCall fused = c;  // the row quantizer reads h (F32) in the residual form
    if (res) {
        fused.x_type = kq::ACT_F32;
        fused.x = norm->hidden;
    }
    if (kq::gemm8_fits(fused) && aligned16(norm->weight)) {
        n.out1 = res ? norm->hidden : nullptr;
        n.w2 = res ? norm->weight : nullptr;
        n.inv_out = inv;
        if (hipError_t e = kq::launch_rms_norm(n, st); e != hipSuccess) return hip_fail(e, "RMS normalization launch");
        fused.norm_inv = inv;
        fused.norm_w1 = norm->weight;
        if (hipError_t e = kq::launch_gemm8(fused, c.act, st); e != hipSuccess) return hip_fail(e, "prefill projection launch");
        return KQ_OK;
    }
    if (kq::gemm_i4_fits(fused) && aligned16(norm->weight)) {
        n.out1 = res ? norm->hidden : nullptr;
        n.w2 = res ? norm->weight : nullptr;
        n.inv_out = inv;
        if (hipError_t e = kq::launch_rms_norm(n, st); e != hipSuccess) return hip_fail(e, "RMS normalization launch");
        c.x = res ? static_cast<const void*>(norm->hidden) : args->x;
        c.x_type = res ? kq::ACT_F32 : c.x_type;
        c.norm_inv = inv;
        c.norm_w1 = norm->weight;
        if (hipError_t e = kq::launch_gemm_i4(c, c.act, st); e != hipSuccess) return hip_fail(e, "prefill projection launch");
        return KQ_OK;
    }
    // Other shapes: the normalized input to the workspace, then the plain projection of it.
    n.out1 = res ? norm->hidden : normed;
    n.w2 = res ? norm->weight : nullptr;
    n.out2 = res ? normed : nullptr;
    if (hipError_t e = kq::launch_rms_norm(n, st); e != hipSuccess) return hip_fail(e, "RMS normalization launch");
    kq_linear_args a = *args;
    a.x = normed;
    a.x_dtype = KQ_F32;
    a.workspace = ws_lin ? base : nullptr;
    a.workspace_bytes = l.lin;
    return gelu_gate ? kq_packed_linear_gelu_gate(weight, &a, stream) : kq_packed_linear(weight, &a, stream);
}

kq_status kq_quantize_weight(const void* weight, kq_dtype dtype, int64_t rows, int64_t cols, int32_t bits,
                             int32_t group_size, int32_t asymmetric_clip, uint8_t* values, float* scales, float* zeros,
                             void* stream) {
    // ops::pack_weight's checks (src/kidi/ops/quantization.cpp:15-20)
    if ((dtype != KQ_F32 && dtype != KQ_F16 && dtype != KQ_BF16) || (bits != 2 && bits != 4 && bits != 8) ||
        group_size <= 0 || group_size % (8 / bits) || rows <= 0 || cols <= 0 || cols % group_size)
        return fail(KQ_INVALID_ARGUMENT, "invalid packed weight dimensions, precision or group size");
    const bool asym = asymmetric_clip != 0 && bits == 4;
    if (!weight || !values || !scales || (asym && !zeros)) return fail(KQ_INVALID_ARGUMENT, "null weight or output");
    const std::size_t elem = dtype == KQ_F32 ? 4 : 2;
    if (reinterpret_cast<std::uintptr_t>(weight) % elem || reinterpret_cast<std::uintptr_t>(scales) % 4 ||
        (asym && reinterpret_cast<std::uintptr_t>(zeros) % 4))
        return fail(KQ_INVALID_ARGUMENT, "misaligned weight, scales or zeros");
    if (rows * (cols / group_size) >= (std::int64_t{1} << 38))  // one thread per (row, group), 2^30 workgroups
        return fail(KQ_UNSUPPORTED, "weight too large for one quantization launch");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (kq_status s = refuse_capture(st, "weight quantization"); s != KQ_OK) return s;
    void* flag = nullptr;
    if (kq_status s = device_scratch(g_pack_scratch, 256, st, &flag); s != KQ_OK) return s;
    int* error = static_cast<int*>(flag);
    if (hipError_t e = hipMemsetAsync(error, 0, sizeof(int), st); e != hipSuccess) return hip_fail(e, "hipMemsetAsync");
    const int dt = dtype == KQ_F32 ? 0 : (dtype == KQ_F16 ? 1 : 2);
    if (hipError_t e = kq::launch_pack_weight(weight, dt, rows, cols, bits, group_size, asym, values, scales, zeros, error, st);
        e != hipSuccess)
        return hip_fail(e, "weight quantization launch");
    int host_error = 0;
    if (hipError_t e = hipMemcpyAsync(&host_error, error, sizeof(int), hipMemcpyDeviceToHost, st); e != hipSuccess)
        return hip_fail(e, "hipMemcpyAsync");
    if (hipError_t e = hipStreamSynchronize(st); e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    if (host_error & 1) return fail(KQ_INVALID_ARGUMENT, "non-finite weight cannot be quantized");
    if (host_error & 2) return fail(KQ_INVALID_ARGUMENT, "quantization scale underflow");
    return KQ_OK;
}

kq_status kq_debug_quantize(const kq_weight* weight, const void* x, kq_dtype x_dtype, int64_t m, float input_scale,
                            int8_t* codes, float* scales, int32_t* sums, int32_t* zero_points, void* stream) {
    kq_linear_args args{};
    args.x = x;
    args.x_dtype = x_dtype;
    args.m = m;
    args.input_scale = input_scale;
    args.y = reinterpret_cast<float*>(codes);  // unused, must be non-null
    kq::LinearCall c;
    std::size_t ws_bytes = 0;
    if (kq_status s = prepare_call(weight, &args, false, c, &ws_bytes); s != KQ_OK) return s;
    if (c.path == kq::PATH_PORTABLE) return fail(KQ_UNSUPPORTED, "the portable path does not quantize activations");
    if (m == 0) return KQ_OK;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    kq::SkinnyPlan plan;
    const bool fused = kq::decode_fits(c);
    if (fused || kq::skinny_plan(c, plan)) {
        // the fused quantizer of the decode projection reports what it computed
        void* ybuf = nullptr;
        if (kq_status s = device_scratch(g_debug_scratch, static_cast<std::size_t>(m * c.w->geo.rows) * 4, st, &ybuf); s != KQ_OK)
            return s;
        c.y = static_cast<float*>(ybuf);
        c.dq_codes = codes;
        c.dq_scales = scales;
        c.dq_sums = sums;
        c.dq_zeros = zero_points;
        const hipError_t e = fused ? kq::launch_decode(c, st) : kq::launch_skinny(c, plan, st);
        if (e != hipSuccess) return hip_fail(e, "debug quantize");
        return KQ_OK;
    }
    void* ws = nullptr;
    if (kq_status s = device_scratch(g_debug_scratch, align_up(ws_bytes) + 256, st, &ws); s != KQ_OK) return s;
    c.act = kq::carve_workspace(*c.w, m, ws);
    if (kq::gemm8_fits(c)) {
        hipError_t e = kq::launch_gemm8(c, c.act, st, true, codes, scales, sums);
        if (e == hipSuccess && zero_points) e = hipMemsetAsync(zero_points, 0, static_cast<std::size_t>(m * (c.w->geo.cols / c.w->geo.group)) * 4, st);
        if (e != hipSuccess) return hip_fail(e, "debug quantize");
        return KQ_OK;
    }
    if (kq::gemm_i4_fits(c)) {
        const hipError_t e = kq::launch_gemm_i4_quantize_dump(c, c.act, codes, scales, sums, zero_points, st);
        if (e != hipSuccess) return hip_fail(e, "debug quantize");
        return KQ_OK;
    }
    if (kq::gemm_i4g_fits(c)) {
        const hipError_t e = kq::launch_gemm_i4g_quantize_dump(c, codes, scales, sums, zero_points, st);
        if (e != hipSuccess) return hip_fail(e, "debug quantize");
        return KQ_OK;
    }
    hipError_t e = kq::launch_quantize(c, st);
    if (e == hipSuccess && codes) e = kq::launch_unpermute_codes(*c.w, c.act, m, codes, st);
    if (e == hipSuccess) e = kq::launch_copy_block_stats(*c.w, c.act, m, scales, sums, zero_points, st);
    if (e != hipSuccess) return hip_fail(e, "debug quantize");
    return KQ_OK;
}

kq_status kq_debug_partials(const kq_weight* weight, const kq_linear_args* args, int32_t* partials, void* stream) {
    kq::LinearCall c;
    std::size_t ws = 0;
    if (kq_status s = prepare_call(weight, args, false, c, &ws); s != KQ_OK) return s;
    if (c.path == kq::PATH_PORTABLE) return fail(KQ_UNSUPPORTED, "the portable path has no integer partials");
    c.dump = partials;
    return run_call(c, args, ws, static_cast<hipStream_t>(stream));
}

kq_status kq_lowbit_parity_linear(const kq_weight* weight, const kq_linear_args* args, void* stream) {
    if (!weight || !args) return fail(KQ_INVALID_ARGUMENT, "null weight or arguments");
    const kq::Weight& w = *as_weight(weight);
    // Context::packed_linear's scale check (ops/context.cpp:824-825), then its LOWBIT_PARITY domain (:919-929)
    if (!std::isfinite(args->input_scale) || args->input_scale < 0 || !std::isfinite(args->output_scale) ||
        args->output_scale < 0)
        return fail(KQ_INVALID_ARGUMENT, "invalid calibrated projection scales");
    if (args->m < 0) return fail(KQ_INVALID_ARGUMENT, "negative row count");
    if (args->x_dtype != KQ_F32 || !(args->input_scale > 0) || !(args->output_scale > 0) ||
        w.scale_type != kq::META_F32 || args->m > INT32_MAX || w.geo.cols > INT32_MAX || w.geo.rows > INT32_MAX)
        return fail(KQ_UNSUPPORTED, "lowbit-parity requires calibrated CPU packed weights with compatible group scales");
    // runtime::parity::packed_linear's scale check (parity_math.cpp:239-240)
    if (!w.scales_positive) return fail(KQ_INVALID_ARGUMENT, "packed weight scales must be finite and positive");
    if (args->m == 0) return KQ_OK;
    if (!args->x || !args->y) return fail(KQ_INVALID_ARGUMENT, "null input or output");
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev != w.device) return fail(KQ_INVALID_ARGUMENT, "weight was packed on another device");
    kq::LinearCall c{};
    c.w = &w;
    c.x = args->x;
    c.x_type = kq::ACT_F32;
    c.M = args->m;
    c.input_scale = args->input_scale;
    c.output_scale = args->output_scale;
    c.y = args->y;
    c.path = kq::PATH_PORTABLE;
    c.parity = true;
    if (hipError_t e = kq::launch_linear(c, static_cast<hipStream_t>(stream)); e != hipSuccess)
        return hip_fail(e, "lowbit-parity projection launch");
    return KQ_OK;
}

int32_t kq_debug_route(const kq_weight* weight, const kq_linear_args* args, int32_t gelu_gate) {
    kq::LinearCall c;
    std::size_t ws = 0;
    if (prepare_call(weight, args, gelu_gate != 0, c, &ws) != KQ_OK) return -1;
    return route_of(c, nullptr);
}

int32_t kq_debug_route_shape(int32_t bits, int32_t group_size, int64_t rows, int64_t cols, int32_t zero_mode,
                             int32_t scale_f16, int64_t m, kq_dtype x_dtype, float input_scale, int32_t gelu_gate) {
    if ((bits != 2 && bits != 4 && bits != 8) || group_size <= 0 || rows <= 0 || cols <= 0 || cols % group_size ||
        group_size % (8 / bits) || zero_mode < kq::ZERO_NONE || zero_mode > kq::ZERO_FLOAT || m < 0 ||
        (x_dtype != KQ_F32 && x_dtype != KQ_BF16) || !std::isfinite(input_scale) || input_scale < 0 ||
        (gelu_gate && rows % 2))
        return -1;
    kq::Weight w;  // geometry and modes only: no device memory is touched
    w.geo = kq::Geometry::make(bits, group_size, rows, cols);
    w.tiled = kq::tiled_group_ok(bits, group_size);
    w.scale_type = scale_f16 ? kq::META_F16 : kq::META_F32;
    w.zero_mode = zero_mode;
    w.has_prefill = kq::gemm8_eligible(w);
    kq::LinearCall c{};
    c.w = &w;
    c.x = nullptr;
    c.x_type = x_dtype == KQ_BF16 ? kq::ACT_BF16 : kq::ACT_F32;
    c.M = m;
    c.input_scale = input_scale;
    c.path = select_path(bits, group_size, cols, rows, zero_mode != kq::ZERO_NONE, input_scale);
    c.gelu_gate = gelu_gate != 0;
    return route_of(c, nullptr);
}

kq_status kq_debug_read_floor(const void* data, size_t bytes, int32_t* sink, void* stream) {
    if (!data || !sink || bytes == 0 || bytes > (std::size_t{1} << 31) || bytes % 16)
        return fail(KQ_INVALID_ARGUMENT, "read floor: device buffer of 16-byte multiple size up to 2 GiB");
    if (hipError_t e = kq::launch_read_floor(data, static_cast<std::uint32_t>(bytes), sink, static_cast<hipStream_t>(stream));
        e != hipSuccess)
        return hip_fail(e, "read floor launch");
    return KQ_OK;
}

kq_status kq_debug_read_floor_shape(const void* data, size_t bytes, int32_t threads, int32_t loads, int32_t empty,
                                    int32_t* sink, void* stream) {
    if (!data || !sink || bytes == 0 || bytes > (std::size_t{1} << 31) || bytes % 16)
        return fail(KQ_INVALID_ARGUMENT, "read floor: device buffer of 16-byte multiple size up to 2 GiB");
    if ((threads != 64 && threads != 128 && threads != 256 && threads != 512 && threads != 1024) ||
        (loads != 1 && loads != 2 && loads != 4 && loads != 8 && loads != 16))
        return fail(KQ_INVALID_ARGUMENT, "read floor: threads 64/128/256/512/1024 and loads 1/2/4/8/16 per lane");
    if (hipError_t e = kq::launch_read_floor_shape(data, static_cast<std::uint32_t>(bytes), threads, loads, empty != 0, sink,
                                                   static_cast<hipStream_t>(stream));
        e != hipSuccess)
        return hip_fail(e, "read floor launch");
    return KQ_OK;
}

int32_t kq_debug_mfma_ceiling_workgroups(void) { return kq::mfma_ceiling_workgroups(); }

kq_status kq_debug_mfma_ceiling(int32_t iterations, int64_t* cycles, int32_t* sink, void* stream) {
    if (!cycles || !sink || iterations <= 0 || iterations > (1 << 24))
        return fail(KQ_INVALID_ARGUMENT, "mfma ceiling: device cycles and sink buffers, 1 to 2^24 iterations");
    if (hipError_t e = kq::launch_mfma_ceiling(iterations, reinterpret_cast<long long*>(cycles), sink, static_cast<hipStream_t>(stream));
        e != hipSuccess)
        return hip_fail(e, "mfma ceiling launch");
    return KQ_OK;
}

size_t kq_layout_bytes(int32_t bits, int32_t group_size, int64_t rows, int64_t cols) {
    if ((bits != 2 && bits != 4 && bits != 8) || rows <= 0 || cols <= 0) return 0;
    return static_cast<size_t>(kq::Geometry::make(bits, group_size, rows, cols).tile_bytes_total());
}

kq_status kq_layout_encode_host(int32_t bits, int64_t rows, int64_t cols, const uint8_t* values, uint8_t* tiles) {
    if ((bits != 2 && bits != 4 && bits != 8) || rows <= 0 || cols <= 0 || cols % (8 / bits) || !values || !tiles)
        return fail(KQ_INVALID_ARGUMENT, "invalid layout arguments");
    kq::encode_tiles(bits, rows, cols, values, tiles);
    return KQ_OK;
}

kq_status kq_layout_decode_host(int32_t bits, int64_t rows, int64_t cols, const uint8_t* tiles, int8_t* codes) {
    if ((bits != 2 && bits != 4 && bits != 8) || rows <= 0 || cols <= 0 || !tiles || !codes)
        return fail(KQ_INVALID_ARGUMENT, "invalid layout arguments");
    kq::decode_tiles(bits, rows, cols, tiles, codes);
    return KQ_OK;
}

}  // extern "C"
