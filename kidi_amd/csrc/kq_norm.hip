// RMS normalization of the quantized linear layer's input (gfx950): Kidi's RMS_NORM / RMS_NORM_RESIDUAL
// (Context::rms_norm / rms_norm_residual, src/kidi/ops/context.cpp:1043-1049, :1103-1122; the CPU RmsNorm operator,
// runtime/ynn/operators.cpp:553-620) and the pieces that fuse it into a projection's activation quantization.
//
//   inv = 1 / sqrt(sum(x^2) / width + epsilon);   plain: y = x * inv * w;   residual: y = (r + x * inv * w) [* s]
//
// The sum of squares has one fixed order on every path of this library (this kernel, the decode projection's fused
// prologue): a row is cut into 512-column segments of 64 pieces of 8 columns (columns past the width read as 0); a
// piece is summed in column order, the 64 pieces of a segment as a balanced pairwise tree in piece order (a
// butterfly over the 64 lanes of a wave: lane l holds piece l, and at each level both partners compute the same
// commutative sum), the segments in order. Fused and standalone forms therefore produce the same bits.
//
// One wave per row, four rows per workgroup. Modes (all fields of NormArgs optional except x, w1):
//   plain:    out1 = x * inv1 * w1, and/or inv_out = inv1                  (RMS_NORM; prefill statistics)
//   residual: h = (r + x * inv1 * w1) [* s] -> out1; with a second weight w2 the projection input of the layer
//             follows: inv2 from h, out2 = h * inv2 * w2 and/or inv_out = inv2
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kq_device.hpp"
#include "kq_internal.hpp"

namespace kq {
namespace {

using namespace dev;

// Eight values of row data starting at column col (bounds-checked per element unless the whole piece is in range
// and the row is 16-byte aligned for vector loads).
__device__ __forceinline__ void load8(const void* base, int f32, std::int64_t row_off, std::int64_t col, std::int64_t width,
                                      bool vec, float (&v)[8]) {
    if (vec && col + 8 <= width) {
        if (f32) {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + row_off + col);
            const float4 a = p[0], b = p[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const std::uint16_t*>(base) + row_off + col);
            const std::uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = __uint_as_float(w4[i] << 16);
                v[2 * i + 1] = __uint_as_float(w4[i] & 0xFFFF0000u);
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = col + i < width ? load_act(base, f32 ? ACT_F32 : ACT_BF16, row_off + col + i) : 0.F;
}

__device__ __forceinline__ void store8(float* base, std::int64_t row_off, std::int64_t col, std::int64_t width, bool vec,
                                       const float (&v)[8]) {
    if (vec && col + 8 <= width) {
        float4* p = reinterpret_cast<float4*>(base + row_off + col);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (col + i < width) base[row_off + col + i] = v[i];
}

// Sum of squares of one 8-column piece in column order, then the segment's butterfly over the wave's 64 lanes.
__device__ __forceinline__ float segment_sum_squares(const float (&v)[8]) {
    float s = v[0] * v[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) s = s + v[i] * v[i];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) s = s + __shfl_xor(s, off);
    return s;
}

struct NormArgs {
    const void* x;         // [rows][width] F32 | BF16
    const void* r;         // residual [rows][width] (x's type), or null (plain form)
    const float* w1;       // [width]
    const float* scale;    // residual form's scalar, or null
    const float* w2;       // second norm's weight (projection input of the residual form), or null
    float* out1;           // plain: normalized x; residual: h
    float* out2;           // residual form: h * inv2 * w2
    float* inv_out;        // per row: inv1 (plain) or inv2 (residual with a second norm)
    std::int64_t rows, width;
    float eps1, eps2;
    int x_f32, vec;
};

__global__ __launch_bounds__(256) void rms_norm_kernel(NormArgs a) {
    const int lane = threadIdx.x & 63;
    const std::int64_t row = static_cast<std::int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;  // whole waves
    const std::int64_t off = row * a.width;
    const bool vec = a.vec != 0;
    const float width_f = static_cast<float>(a.width);
    float total = 0.F;
    for (std::int64_t seg = 0; seg * 512 < a.width; ++seg) {
        float v[8];
        load8(a.x, a.x_f32, off, seg * 512 + 8 * lane, a.width, vec, v);
        const float s = segment_sum_squares(v);
        total = seg == 0 ? s : total + s;
    }
    const float inv1 = 1.F / sqrtf(total / width_f + a.eps1);
    if (!a.r) {
        if (a.inv_out && lane == 0) a.inv_out[row] = inv1;
        if (!a.out1) return;
        for (std::int64_t seg = 0; seg * 512 < a.width; ++seg) {
            const std::int64_t col = seg * 512 + 8 * lane;
            float v[8], w[8];
            load8(a.x, a.x_f32, off, col, a.width, vec, v);
            load8(a.w1, 1, 0, col, a.width, vec, w);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = v[i] * inv1 * w[i];
            store8(a.out1, off, col, a.width, vec, v);
        }
        return;
    }
    const bool scaled = a.scale != nullptr;
    const float s = scaled ? a.scale[0] : 1.F;
    const bool second = a.w2 != nullptr || a.inv_out != nullptr;
    // h of one piece, computed the same way in both passes below
    auto hidden = [&](std::int64_t col, float (&h)[8]) {
        float v[8], w[8];
        load8(a.x, a.x_f32, off, col, a.width, vec, v);
        load8(a.r, a.x_f32, off, col, a.width, vec, h);
        load8(a.w1, 1, 0, col, a.width, vec, w);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            h[i] = h[i] + v[i] * inv1 * w[i];
            if (scaled) h[i] = h[i] * s;
        }
    };
    float total2 = 0.F;
    for (std::int64_t seg = 0; seg * 512 < a.width; ++seg) {
        const std::int64_t col = seg * 512 + 8 * lane;
        float h[8];
        hidden(col, h);
        if (a.out1) store8(a.out1, off, col, a.width, vec, h);
        if (second) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (col + i >= a.width) h[i] = 0.F;
            const float t = segment_sum_squares(h);
            total2 = seg == 0 ? t : total2 + t;
        }
    }
    if (!second) return;
    const float inv2 = 1.F / sqrtf(total2 / width_f + a.eps2);
    if (a.inv_out && lane == 0) a.inv_out[row] = inv2;
    if (!a.out2) return;
    for (std::int64_t seg = 0; seg * 512 < a.width; ++seg) {
        const std::int64_t col = seg * 512 + 8 * lane;
        float h[8], w[8];
        hidden(col, h);
        load8(a.w2, 1, 0, col, a.width, vec, w);
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = h[i] * inv2 * w[i];
        store8(a.out2, off, col, a.width, vec, h);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t launch_rms_norm(const NormLaunch& n, hipStream_t stream) {
    if (n.rows == 0) return hipSuccess;
    NormArgs a{};
    a.x = n.x;
    a.r = n.residual;
    a.w1 = n.w1;
    a.scale = n.scale;
    a.w2 = n.w2;
    a.out1 = n.out1;
    a.out2 = n.out2;
    a.inv_out = n.inv_out;
    a.rows = n.rows;
    a.width = n.width;
    a.eps1 = n.eps1;
    a.eps2 = n.eps2;
    a.x_f32 = n.x_type == ACT_F32;
    // vector loads and stores need every row start 16-byte aligned: width % 8 == 0 covers both element sizes
    bool vec = n.width % 8 == 0;
    for (const void* p : {n.x, n.residual, static_cast<const void*>(n.w1), static_cast<const void*>(n.w2),
                          static_cast<const void*>(n.out1), static_cast<const void*>(n.out2)})
        if (p && !aligned16(p)) vec = false;
    a.vec = vec;
    const dim3 grid(static_cast<unsigned>((n.rows + 3) / 4)), block(256);
    hipLaunchKernelGGL(rms_norm_kernel, grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace kq
