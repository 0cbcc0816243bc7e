// Device-side pieces shared by the kernels of the quantized linear layer (gfx950): operand helpers, the activation
// quantizer's arithmetic, the tile-slot unpacking and the kernel argument block.
//
// Float code is compiled without contraction (-ffp-contract=off), so every a*b+c below rounds twice, as the
// reference's C++ does; divisions are IEEE correctly rounded (HIP's default, no fast-math).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kq_internal.hpp"

namespace kq {
namespace dev {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float meta_load(const float* p, std::int64_t i) { return p[i]; }
__device__ __forceinline__ float meta_load(const __half* p, std::int64_t i) { return __half2float(p[i]); }

__device__ __forceinline__ float bf16_bits(std::uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float load_act(const void* x, int type, std::int64_t i) {
    if (type == ACT_BF16) return bf16_bits(static_cast<std::uint32_t>(static_cast<const std::uint16_t*>(x)[i]));
    return static_cast<const float*>(x)[i];
}

// Four consecutive activations starting at element i (i % 4 == 0): one 8-byte (bf16) or 16-byte (f32) load.
__device__ __forceinline__ void load_act4(const void* x, int type, std::int64_t i, float (&v)[4]) {
    if (type == ACT_BF16) {
        const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const std::uint16_t*>(x) + i);
        v[0] = bf16_bits(r.x & 0xFFFFu);
        v[1] = bf16_bits(r.x >> 16);
        v[2] = bf16_bits(r.y & 0xFFFFu);
        v[3] = bf16_bits(r.y >> 16);
    } else {
        const float4 r = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + i);
        v[0] = r.x;
        v[1] = r.y;
        v[2] = r.z;
        v[3] = r.w;
    }
}

// min(max(v, lo), hi) for finite or infinite v in one v_med3_f32 (activations are finite by contract).
__device__ __forceinline__ float clampf(float v, float lo, float hi) { return __builtin_amdgcn_fmed3f(v, lo, hi); }

// Static output rounding (eager_test.cpp:100-102): clamp(rint(y / out), -128, 127) * out when out > 0.
__device__ __forceinline__ float calibrate_output(float v, float out) {
    return out > 0.F ? clampf(__builtin_rintf(v / out), -128.F, 127.F) * out : v;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Streaming 16-byte weight load (each weight byte is read once per projection).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float gelu_tanh(float g) {
    const float inner = 0.7978845608028654F * (g + 0.044715F * g * g * g);
    return 0.5F * g * (1.F + tanhf(inner));
}

// ---------------------------------------------------------------------------------------------------------------
// Activation quantizer arithmetic, per (row, K-block) with block statistics mx (max, or max |x| for mode 0) and mn:
//   QUANT_DYN_SYM  (2/4-bit weights), hnsw_test.cpp:513-520: s = max/127, inverse = 127/max,
//                  q = clamp(rint(x * inverse), -127, 127); an all-zero block gives codes 0 and s = 0.
//   QUANT_DYN_ASYM (8-bit weights), hnsw_test.cpp:492-511: rmin = min(0, x), rmax = max(0, x),
//                  inverse = 255/(rmax - rmin), s = (rmax - rmin)/255, XNNPACK zero point
//                  zp = rint(clamp(fzp, -128, 127)), q = clamp(round(x * inverse) + zp, -128, 127) (std::round).
//   QUANT_STATIC   (calibrated), eager_test.cpp:97-98: q = clamp(rint(x / input_scale), -128, 127).
// Blocks outside the real rows/columns (tile padding) report scale 0 and zero point 0; their codes are 0.
enum QuantMode : int { QUANT_DYN_SYM = 0, QUANT_DYN_ASYM = 1, QUANT_STATIC = 2 };

struct QuantBlock {
    float s = 0.F, inverse = 0.F;
    int zp = 0;
    bool nonzero = false;  // QUANT_DYN_SYM: max > 0
};

__device__ __forceinline__ QuantBlock quant_block(int mode, float mx, float mn, float input_scale, bool live) {
    QuantBlock p;
    if (mode == QUANT_DYN_SYM) {
        if (mx > 0.F) {
            p.inverse = 127.F / mx;
            p.s = mx / 127.F;
            p.nonzero = true;
        }
    } else if (mode == QUANT_DYN_ASYM) {
        const float rdiff = mx - mn;
        p.inverse = rdiff > 0.F ? 255.F / rdiff : 0.F;
        p.s = rdiff > 0.F ? rdiff / 255.F : 1.F;
        const float min_error = -128.F + mn * p.inverse;
        const float max_error = 127.F + mx * p.inverse;
        const float fzp = min_error + max_error > 0.F ? -128.F - mn * p.inverse : 127.F - mx * p.inverse;
        p.zp = rdiff > 0.F ? static_cast<int>(__builtin_rintf(clampf(fzp, -128.F, 127.F))) : -128;
    } else {
        p.s = input_scale;
    }
    if (!live) {
        p.s = 0.F;
        p.zp = 0;
    }
    return p;
}

__device__ __forceinline__ int quant_code(int mode, float v, const QuantBlock& p, float input_scale) {
    if (mode == QUANT_DYN_SYM) return p.nonzero ? static_cast<int>(clampf(__builtin_rintf(v * p.inverse), -127.F, 127.F)) : 0;
    if (mode == QUANT_DYN_ASYM) {
        const int code = static_cast<int>(roundf(v * p.inverse)) + p.zp;
        return code < -128 ? -128 : (code > 127 ? 127 : code);
    }
    return static_cast<int>(clampf(__builtin_rintf(v / input_scale), -128.F, 127.F));
}

// Block statistics accumulation: mode QUANT_DYN_SYM tracks max |x|, QUANT_DYN_ASYM tracks min(0, x) and max(0, x).
__device__ __forceinline__ void quant_stat(int mode, float v, float& mx, float& mn) {
    if (mode == QUANT_DYN_ASYM) {
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    } else {
        mx = fmaxf(mx, fabsf(v));
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Tile shapes and slot unpacking.

template <int BITS>
struct TileShape {
    static constexpr int KT = 512 / BITS;  // columns per tile
    static constexpr int J = KT / 64;      // 64-column blocks per tile
    static constexpr int CH = 2 * J;       // 32-column chunks per tile
};

// Codes of 64-column block j of a lane's 16-byte slot, as 4 dwords of int8 lanes in activation order.
template <int BITS, int j>
__device__ __forceinline__ void unpack_block(const uint4 w, int (&o)[4]) {
    if constexpr (BITS == 8) {
        o[0] = static_cast<int>(w.x);
        o[1] = static_cast<int>(w.y);
        o[2] = static_cast<int>(w.z);
        o[3] = static_cast<int>(w.w);
    } else if constexpr (BITS == 4) {
        const std::uint32_t a = j == 0 ? w.x : w.z;
        const std::uint32_t b = j == 0 ? w.y : w.w;
        o[0] = static_cast<int>(a & 0x0F0F0F0Fu);
        o[1] = static_cast<int>((a >> 4) & 0x0F0F0F0Fu);
        o[2] = static_cast<int>(b & 0x0F0F0F0Fu);
        o[3] = static_cast<int>((b >> 4) & 0x0F0F0F0Fu);
    } else {
        const std::uint32_t a = j == 0 ? w.x : (j == 1 ? w.y : (j == 2 ? w.z : w.w));
        o[0] = static_cast<int>(a & 0x03030303u);
        o[1] = static_cast<int>((a >> 2) & 0x03030303u);
        o[2] = static_cast<int>((a >> 4) & 0x03030303u);
        o[3] = static_cast<int>((a >> 6) & 0x03030303u);
    }
}

// Runtime-j form for loops the compiler fully unrolls.
template <int BITS>
__device__ __forceinline__ void unpack_block_j(const uint4 w, int j, int (&o)[4]) {
    if constexpr (BITS == 8) {
        unpack_block<8, 0>(w, o);
    } else if constexpr (BITS == 4) {
        if (j == 0) unpack_block<4, 0>(w, o);
        else unpack_block<4, 1>(w, o);
    } else {
        if (j == 0) unpack_block<2, 0>(w, o);
        else if (j == 1) unpack_block<2, 1>(w, o);
        else if (j == 2) unpack_block<2, 2>(w, o);
        else unpack_block<2, 3>(w, o);
    }
}

// Zero-point nibble of row nn (0..15) of one (tile, group) record of 8 bytes.
__device__ __forceinline__ int zero_point_at(const std::uint8_t* zp, std::int64_t meta_index, int nn) {
    return (zp[(meta_index - nn) / 2 + nn / 2] >> (4 * (nn & 1))) & 15;
}

// ---------------------------------------------------------------------------------------------------------------
// Kernel argument block.
struct LinearArgs {
    const void* x;                // raw activations
    int x_type;
    const std::uint8_t* tiles;
    const void* scales;
    const std::uint8_t* zero_points;
    const void* zeros;
    const std::int32_t* code_sums;
    const std::int8_t* q;
    const float* a_scale;
    const std::int32_t* a_sum;
    const std::int32_t* a_zero;
    float* y;
    std::int32_t* dump;
    std::int64_t M, N, K, cols_p, k_tiles, n_tiles;
    int group, groups_p, groups;  // groups = K / g (real)
    int zero_mode, zero_half, is_static, gelu;
    int parity;                   // portable kernel: LOWBIT_PARITY form (serial FMA, zeros not applied)
    float input_scale, output_scale;
    int units, tiles_per_unit;    // GEMV split of the K range across waves
    // skinny (fused quantization) projection
    int quant_mode, scale_half;
    int chunk_tiles;              // tiles quantized and staged per chunk (a multiple of the tiles per group)
    int wave_lds;                 // LDS bytes per wave
    int off_stats, off_meta;      // byte offsets inside a wave's LDS region
    int off_x2, off_w;            // ... of the second metadata words and of the staged weight tiles
    int scale_block, x2_block;    // LDS bytes per row tile of a chunk's raw scales / second words
    int red_off;                  // byte offset of the cross-wave reduction buffer
    int lg_group, lg_chunk_cols, lg_waves, lg_tiles_per_unit;  // log2 of g, of the chunk's columns, of W, of tiles/group
    std::int8_t* dq_codes;        // optional dumps of the fused quantizer (natural order [M][K], [M][K/g])
    float* dq_scales;
    std::int32_t* dq_sums;
    std::int32_t* dq_zeros;
};

// Kernel arguments of a prepared call (kq_kernels.hip).
LinearArgs make_linear_args(const LinearCall& c);

}  // namespace dev
}  // namespace kq
