// HIP kernels of the MI355X quantized linear layer (gfx950). Build: hipcc --offload-arch=gfx950 -ffp-contract=off.
//
// Kernels:
//   quantize_tiled     dynamic/calibrated activation quantization into the permuted code order of the tiles
//   gemv_kernel        decode projection, M <= 8: 128-bit tile loads, v_dot4_i32_i8 on unpacked codes, exact
//                      int32 per-group partials reduced across lanes, fp32 group epilogue, LDS cross-wave sum
//   gemm_kernel        prefill projection, M > 8: LDS-staged int8 activation and packed weight tiles,
//                      v_mfma_i32_16x16x64_i8 / 16x16x32_i8 per group, fp32 epilogue per group
//   rowmajor kernels   group sizes the tiles cannot carry (Kidi's own layout, exact integer per group)
//   portable_kernel    Kidi's portable float path (small N, no dynamic 2-bit, calibrated with zeros)
//
// Numerics follow Kidi's CPU operators (runtime/ynn/operators.cpp:1036-1319, :2639-2713) as restated in the
// closed forms cited at each kernel. Float code is compiled without contraction so every a*b+c below rounds
// twice, as the reference's C++ does; divisions are IEEE correctly rounded (HIP's default).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kq_device.hpp"
#include "kq_internal.hpp"

namespace kq {
namespace {

using namespace dev;


// ---------------------------------------------------------------------------------------------------------------
// Activation quantization into a workspace (used ahead of the prefill GEMM, M > 16). One group of g columns is
// handled by T = g/8 lanes (T a power of two up to 64; larger groups loop), each lane owning 8-column chunks whose
// codes land at act_position(k0). Arithmetic: quant_block / quant_code (kq_device.hpp).
// Rows >= M and columns >= K (tile padding) get codes 0, scale 0, sum 0, zero point 0.
struct QuantArgs {
    const void* x;
    int x_type;
    std::int64_t M, K, cols_p, rows_p;
    int group, groups_p, lanes;
    float input_scale;
    std::int8_t* q;
    float* scale;
    std::int32_t* sum;
    std::int32_t* zero;
    int permuted;  // 1: tiled code order, 0: natural order
};

template <int MODE>
__global__ __launch_bounds__(256) void quantize_kernel(QuantArgs a) {
    const int lane = threadIdx.x & 63;
    const std::int64_t wave = (static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int T = a.lanes;
    const std::int64_t gid = wave * (64 / T) + lane / T;
    const int sub = lane % T;
    const bool valid = gid < a.rows_p * a.groups_p;
    const std::int64_t m = valid ? gid / a.groups_p : 0;
    const int b = valid ? static_cast<int>(gid % a.groups_p) : 0;
    const int chunks = a.group / 8;
    const bool live_row = valid && m < a.M;

    // pass 1: block statistics
    float mx = 0.F, mn = 0.F;
    for (int c = sub; c < chunks; c += T) {
        const std::int64_t k0 = static_cast<std::int64_t>(b) * a.group + 8 * c;
        if (!live_row || k0 >= a.K) continue;
#pragma unroll
        for (int i = 0; i < 8; ++i) quant_stat(MODE, load_act(a.x, a.x_type, m * a.K + k0 + i), mx, mn);
    }
    for (int off = T / 2; off >= 1; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off));
        if (MODE == QUANT_DYN_ASYM) mn = fminf(mn, __shfl_xor(mn, off));
    }
    const bool live_block = live_row && static_cast<std::int64_t>(b) * a.group < a.K;
    const QuantBlock p = quant_block(MODE, mx, mn, a.input_scale, live_block);

    // pass 2: codes
    int total = 0;
    for (int c = sub; c < chunks; c += T) {
        const std::int64_t k0 = static_cast<std::int64_t>(b) * a.group + 8 * c;
        if (!valid) continue;
        std::uint32_t lo = 0, hi = 0;
        if (live_row && k0 < a.K) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int code = quant_code(MODE, load_act(a.x, a.x_type, m * a.K + k0 + i), p, a.input_scale);
                total += code;
                const std::uint32_t byte = static_cast<std::uint32_t>(code) & 0xFFu;
                if (i < 4) lo |= byte << (8 * i);
                else hi |= byte << (8 * (i - 4));
            }
        }
        if (a.permuted) {
            *reinterpret_cast<uint2*>(a.q + m * a.cols_p + act_position(k0)) = make_uint2(lo, hi);
        } else if (k0 < a.K) {
            std::int8_t* dst = a.q + m * a.K + k0;
#pragma unroll
            for (int i = 0; i < 8; ++i) dst[i] = static_cast<std::int8_t>(((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xFF);
        }
    }
    for (int off = T / 2; off >= 1; off >>= 1) total += __shfl_xor(total, off);
    if (valid && sub == 0) {
        const std::int64_t o = m * a.groups_p + b;
        a.scale[o] = p.s;
        a.sum[o] = total;
        a.zero[o] = p.zp;
    }
}

// Natural-order quantization for arbitrary group sizes (one thread per block; used with the row-major layout).
template <int MODE>
__global__ __launch_bounds__(256) void quantize_rowmajor_kernel(QuantArgs a) {
    const std::int64_t gid = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::int64_t blocks = a.K / a.group;
    if (gid >= a.M * blocks) return;
    const std::int64_t m = gid / blocks, b = gid % blocks;
    const std::int64_t base = m * a.K + b * a.group;
    float mx = 0.F, mn = 0.F;
    for (int c = 0; c < a.group; ++c) quant_stat(MODE, load_act(a.x, a.x_type, base + c), mx, mn);
    const QuantBlock p = quant_block(MODE, mx, mn, a.input_scale, true);
    int total = 0;
    for (int c = 0; c < a.group; ++c) {
        const int code = quant_code(MODE, load_act(a.x, a.x_type, base + c), p, a.input_scale);
        a.q[base + c] = static_cast<std::int8_t>(code);
        total += code;
    }
    a.scale[gid] = p.s;
    a.sum[gid] = total;
    a.zero[gid] = p.zp;
}

// Integer partial of one finished group -> exact int32 partial P' and its fp32 contribution.
//   2/4-bit:   P' = sum q*u - zp*Q  (u = c + 2^(b-1); zp = 2^(b-1) symmetric / additive zeros, zero point else)
//   8-bit:     P' = sum q*c - zp_a*C  (zp_a = 0 calibrated)
//   t = s * P' (+ z * Q for additive zeros); acc += a_s * t (dynamic) or acc += t (calibrated, * input_scale later)
// This is the closed form y = sum_b a_s (w_s P + w_z Q) of BlockwiseLinear (operators.cpp:1118-1169) with
// w_z = (8 - zp) w_s folded into the integer partial.
template <int BITS, typename ST>
__device__ __forceinline__ float group_term(const LinearArgs& a, std::int64_t meta, std::int64_t m, int b, int P,
                                            int nn, std::int64_t n, float acc) {
    const std::int64_t ab = m * a.groups_p + b;
    const float s = meta_load(static_cast<const ST*>(a.scales), meta);
    int Pp;
    float zf = 0.F;
    if constexpr (BITS == 8) {
        Pp = a.is_static ? P : P - a.a_zero[ab] * a.code_sums[meta];
    } else {
        int zw = sign_offset(BITS);
        if (a.zero_mode == ZERO_POINT) {
            const std::int64_t zi = (meta - nn) / 2 + nn / 2;  // 8 bytes per (tile, group)
            zw = (a.zero_points[zi] >> (4 * (nn & 1))) & 15;
        }
        Pp = P - zw * a.a_sum[ab];
        if (a.zero_mode == ZERO_FLOAT)
            zf = a.zero_half ? __half2float(static_cast<const __half*>(a.zeros)[meta]) : static_cast<const float*>(a.zeros)[meta];
    }
    if (a.dump && b < a.groups && n < a.N && m < a.M) a.dump[(m * a.N + n) * a.groups + b] = Pp;
    float t = s * static_cast<float>(Pp);
    if (BITS != 8 && a.zero_mode == ZERO_FLOAT) t = t + zf * static_cast<float>(a.a_sum[ab]);
    return a.is_static ? acc + t : acc + a.a_scale[ab] * t;
}


// ---------------------------------------------------------------------------------------------------------------
// Decode GEMV (M <= 8). Grid: one workgroup per 16-row tile (two with gelu gating: gate tile and its up tile);
// W waves split the K range into whole groups (g >= KT) or tiles (g < KT). Per tile a lane issues one 16-byte
// weight load and J 16-byte activation loads per row; partials of each 32-column chunk are sums of 8 products
// per lane (two v_dot4) and are reduced across the chunk's 4 lanes (xor 16, xor 32) when a group completes.
template <int BITS, int M, typename ST, int U>
__global__ __launch_bounds__(1024) void gemv_kernel(LinearArgs a) {
    using TS = TileShape<BITS>;
    constexpr int KT = TS::KT, J = TS::J, CH = TS::CH;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int nn = lane & 15, L = lane >> 4;
    const std::int64_t nt = blockIdx.x;
    const std::int64_t n = nt * kTileRows + nn;
    const int u0 = static_cast<int>(static_cast<std::int64_t>(wave) * a.units / waves);
    const int u1 = static_cast<int>(static_cast<std::int64_t>(wave + 1) * a.units / waves);
    const int t0 = u0 * a.tiles_per_unit, t1 = u1 * a.tiles_per_unit;
    const bool wide = a.group >= KT;            // a group spans whole tiles
    const int chunks_per_group = a.group / 32;  // when !wide
    const uint4* wbase = reinterpret_cast<const uint4*>(a.tiles + nt * a.k_tiles * kTileBytes) + lane;

    float acc[M];
    int gacc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        acc[m] = 0.F;
        gacc[m] = 0;
    }

    for (int tb = t0; tb < t1; tb += U) {
        uint4 wv[U];
        uint4 qv[U][M][J];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + u;
            if (t < t1) {
                wv[u] = load_stream(wbase + static_cast<std::int64_t>(t) * 64);
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int j = 0; j < J; ++j)
                        qv[u][m][j] = *reinterpret_cast<const uint4*>(a.q + m * a.cols_p + static_cast<std::int64_t>(t) * KT + 64 * j + 16 * L);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + u;
            if (t >= t1) break;
            int cp[M][CH];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                int o[4];
                if constexpr (J == 1) unpack_block<BITS, 0>(wv[u], o);
                else if constexpr (J == 2) {
                    if (j == 0) unpack_block<BITS, 0>(wv[u], o);
                    else unpack_block<BITS, 1>(wv[u], o);
                } else {
                    if (j == 0) unpack_block<BITS, 0>(wv[u], o);
                    else if (j == 1) unpack_block<BITS, 1>(wv[u], o);
                    else if (j == 2) unpack_block<BITS, 2>(wv[u], o);
                    else unpack_block<BITS, 3>(wv[u], o);
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint4 qq = qv[u][m][j];
                    cp[m][2 * j] = sdot4(o[1], static_cast<int>(qq.y), sdot4(o[0], static_cast<int>(qq.x), 0));
                    cp[m][2 * j + 1] = sdot4(o[3], static_cast<int>(qq.w), sdot4(o[2], static_cast<int>(qq.z), 0));
                }
            }
            if (wide) {
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int c = 0; c < CH; ++c) gacc[m] += cp[m][c];
                if ((t + 1) % a.tiles_per_unit == 0 || a.tiles_per_unit == 1) {
                    const int b = t / (a.group / KT);
                    const std::int64_t meta = (nt * a.groups_p + b) * kTileRows + nn;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        int P = gacc[m];
                        P += __shfl_xor(P, 16);
                        P += __shfl_xor(P, 32);
                        acc[m] = group_term<BITS, ST>(a, meta, m, b, P, nn, n, acc[m]);
                        gacc[m] = 0;
                    }
                }
            } else {
                const int gpt = KT / a.group;
                for (int gi = 0; gi < gpt; ++gi) {
                    const int b = t * gpt + gi;
                    const std::int64_t meta = (nt * a.groups_p + b) * kTileRows + nn;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        int P = 0;
#pragma unroll
                        for (int c = 0; c < CH; ++c)
                            if (c / chunks_per_group == gi) P += cp[m][c];
                        P += __shfl_xor(P, 16);
                        P += __shfl_xor(P, 32);
                        acc[m] = group_term<BITS, ST>(a, meta, m, b, P, nn, n, acc[m]);
                    }
                }
            }
        }
    }

    // cross-wave reduction: every lane of a row holds the same accumulator; lanes L == 0 publish
    __shared__ float red[16][8][kTileRows];
    if (L == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) red[wave][m][nn] = acc[m];
    }
    __syncthreads();
    if (wave == 0 && L == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float v = 0.F;
            for (int w = 0; w < waves; ++w) v = v + red[w][m][nn];
            if (a.is_static) v = v * a.input_scale;
            v = calibrate_output(v, a.output_scale);
            if (m < a.M && n < a.N) a.y[m * a.N + n] = v;
        }
    }
}

// GEMV with GELU-tanh gating: one workgroup computes the gate tile and the matching up tile, so the product
// never leaves registers. Rows [0, I) are gate, [I, 2I) up (Kidi's gate_up_proj, model/gemma4.cpp:308-316).
template <int BITS, int M, typename ST, int U>
__global__ __launch_bounds__(1024) void gemv_gelu_kernel(LinearArgs a) {
    using TS = TileShape<BITS>;
    constexpr int KT = TS::KT, J = TS::J, CH = TS::CH;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int nn = lane & 15, L = lane >> 4;
    const std::int64_t half_tiles = a.n_tiles / 2;
    const std::int64_t nt_g = blockIdx.x, nt_u = blockIdx.x + half_tiles;
    const std::int64_t half_n = a.N / 2;
    const int u0 = static_cast<int>(static_cast<std::int64_t>(wave) * a.units / waves);
    const int u1 = static_cast<int>(static_cast<std::int64_t>(wave + 1) * a.units / waves);
    const int t0 = u0 * a.tiles_per_unit, t1 = u1 * a.tiles_per_unit;
    const bool wide = a.group >= KT;
    const int chunks_per_group = a.group / 32;
    const uint4* wg = reinterpret_cast<const uint4*>(a.tiles + nt_g * a.k_tiles * kTileBytes) + lane;
    const uint4* wu = reinterpret_cast<const uint4*>(a.tiles + nt_u * a.k_tiles * kTileBytes) + lane;

    float acc[2][M];
    int gacc[2][M];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            acc[s][m] = 0.F;
            gacc[s][m] = 0;
        }
    for (int tb = t0; tb < t1; tb += U) {
        uint4 wv[2][U];
        uint4 qv[U][M][J];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + u;
            if (t < t1) {
                wv[0][u] = load_stream(wg + static_cast<std::int64_t>(t) * 64);
                wv[1][u] = load_stream(wu + static_cast<std::int64_t>(t) * 64);
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int j = 0; j < J; ++j)
                        qv[u][m][j] = *reinterpret_cast<const uint4*>(a.q + m * a.cols_p + static_cast<std::int64_t>(t) * KT + 64 * j + 16 * L);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = tb + u;
            if (t >= t1) break;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const std::int64_t nt = s ? nt_u : nt_g;
                const std::int64_t n = nt * kTileRows + nn;
                int cp[M][CH];
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    int o[4];
                    if constexpr (J == 1) unpack_block<BITS, 0>(wv[s][u], o);
                    else if constexpr (J == 2) {
                        if (j == 0) unpack_block<BITS, 0>(wv[s][u], o);
                        else unpack_block<BITS, 1>(wv[s][u], o);
                    } else {
                        if (j == 0) unpack_block<BITS, 0>(wv[s][u], o);
                        else if (j == 1) unpack_block<BITS, 1>(wv[s][u], o);
                        else if (j == 2) unpack_block<BITS, 2>(wv[s][u], o);
                        else unpack_block<BITS, 3>(wv[s][u], o);
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const uint4 qq = qv[u][m][j];
                        cp[m][2 * j] = sdot4(o[1], static_cast<int>(qq.y), sdot4(o[0], static_cast<int>(qq.x), 0));
                        cp[m][2 * j + 1] = sdot4(o[3], static_cast<int>(qq.w), sdot4(o[2], static_cast<int>(qq.z), 0));
                    }
                }
                if (wide) {
#pragma unroll
                    for (int m = 0; m < M; ++m)
#pragma unroll
                        for (int c = 0; c < CH; ++c) gacc[s][m] += cp[m][c];
                    if ((t + 1) % a.tiles_per_unit == 0 || a.tiles_per_unit == 1) {
                        const int b = t / (a.group / KT);
                        const std::int64_t meta = (nt * a.groups_p + b) * kTileRows + nn;
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            int P = gacc[s][m];
                            P += __shfl_xor(P, 16);
                            P += __shfl_xor(P, 32);
                            acc[s][m] = group_term<BITS, ST>(a, meta, m, b, P, nn, n, acc[s][m]);
                            gacc[s][m] = 0;
                        }
                    }
                } else {
                    const int gpt = KT / a.group;
                    for (int gi = 0; gi < gpt; ++gi) {
                        const int b = t * gpt + gi;
                        const std::int64_t meta = (nt * a.groups_p + b) * kTileRows + nn;
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            int P = 0;
#pragma unroll
                            for (int c = 0; c < CH; ++c)
                                if (c / chunks_per_group == gi) P += cp[m][c];
                            P += __shfl_xor(P, 16);
                            P += __shfl_xor(P, 32);
                            acc[s][m] = group_term<BITS, ST>(a, meta, m, b, P, nn, n, acc[s][m]);
                        }
                    }
                }
            }
        }
    }
    __shared__ float red[16][2][8][kTileRows];
    if (L == 0) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int m = 0; m < M; ++m) red[wave][s][m][nn] = acc[s][m];
    }
    __syncthreads();
    if (wave == 0 && L == 0) {
        const std::int64_t i = nt_g * kTileRows + nn;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float g = 0.F, up = 0.F;
            for (int w = 0; w < waves; ++w) {
                g = g + red[w][0][m][nn];
                up = up + red[w][1][m][nn];
            }
            if (a.is_static) {
                g = g * a.input_scale;
                up = up * a.input_scale;
            }
            g = calibrate_output(g, a.output_scale);
            up = calibrate_output(up, a.output_scale);
            if (m < a.M && i < half_n) a.y[m * half_n + i] = gelu_tanh(g) * up;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Prefill GEMM (M > 8). Workgroup tile 128 rows x 128 columns (8 weight tiles), 4 waves of 64 x 64. Per k-tile the
// workgroup stages the int8 activation rows (row stride KT + 16 bytes to spread LDS banks) and the 8 packed
// weight tiles in LDS plus the group metadata; each wave unpacks its 4 weight slots once per tile and runs
// 16x16x64 int8 MFMAs (16x16x32 per 32-column group when g = 32) into per-group int32 accumulators, which the
// group epilogue folds into fp32 accumulators (group_term arithmetic, per element). With GELU gating the 8 tiles
// are 4 gate tiles and the 4 matching up tiles, and every wave holds 2 gate + 2 up subtiles of the same columns.
constexpr int GM = 128, GN = 128;

// Group metadata of one k-tile: at most KT/32 groups close in a tile. Arrays a mode never reads keep one slot.
template <int BITS>
struct GemmMeta {
    static constexpr int G = 512 / BITS / 32;
    static constexpr int GZ = BITS == 4 ? G : 1;  // additive float zeros (4-bit only)
    static constexpr int G8 = BITS == 8 ? G : 1;  // activation zero points and code sums (8-bit only)
    float a_s[G][GM];
    int a_q[G][GM];
    int a_z[G8][GM];
    float s[G][GN];
    int zw[G][GN];
    float zf[GZ][GN];
    int cs[G8][GN];
};

// LDS tile slot (0..7) of wave column wn, subtile ni.
__device__ __forceinline__ int gemm_slot(bool gelu, int wn, int ni) {
    return gelu ? (ni < 2 ? 2 * wn + ni : 4 + 2 * wn + ni - 2) : 4 * wn + ni;
}

template <int BITS, typename ST>
__global__ __launch_bounds__(256) void gemm_kernel(LinearArgs a) {
    using TS = TileShape<BITS>;
    constexpr int KT = TS::KT, J = TS::J;
    constexpr int AS = KT + 16;  // LDS row stride of the activation tile
    __shared__ __attribute__((aligned(16))) std::int8_t lds_a[GM * AS];
    __shared__ __attribute__((aligned(16))) std::uint8_t lds_b[8 * kTileBytes];
    __shared__ GemmMeta<BITS> meta;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int L = lane >> 4, col = lane & 15;
    const bool gelu = a.gelu != 0;

    // XCD-aware order: consecutive workgroups land on different XCDs; give each XCD a contiguous slab of tiles
    const std::int64_t half_tiles = a.n_tiles / 2;
    const std::int64_t m_blocks = (a.M + GM - 1) / GM;
    const std::int64_t n_blocks = gelu ? (half_tiles + 3) / 4 : (a.n_tiles + 7) / 8;
    const std::int64_t total = m_blocks * n_blocks;
    std::int64_t bid = blockIdx.x;
    if (total % 8 == 0) bid = (bid % 8) * (total / 8) + bid / 8;
    const std::int64_t nb = bid % n_blocks, mb = bid / n_blocks;
    const std::int64_t m0 = mb * GM;
    // global weight tile of LDS slot t (n_tiles when out of range)
    auto slot_tile = [&](int t) -> std::int64_t {
        if (gelu) {
            const std::int64_t g = nb * 4 + (t & 3);
            return g < half_tiles ? (t < 4 ? g : half_tiles + g) : a.n_tiles;
        }
        const std::int64_t nt = nb * 8 + t;
        return nt < a.n_tiles ? nt : a.n_tiles;
    };

    const int gpt = a.group >= KT ? 1 : KT / a.group;  // groups per tile
    const int tiles_per_group = a.group >= KT ? a.group / KT : 1;

    v4i acc_i[4][4];
    float acc_f[4][4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc_i[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int r = 0; r < 4; ++r) acc_f[i][j][r] = 0.F;
        }

    auto epilogue = [&](int gi, int b) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int cl = gemm_slot(gelu, wn, ni) * 16 + col;
            const float s = meta.s[gi][cl];
            const int zw = meta.zw[gi][cl];
            const float zf = BITS == 4 ? meta.zf[BITS == 4 ? gi : 0][cl] : 0.F;
            const int cs = BITS == 8 ? meta.cs[BITS == 8 ? gi : 0][cl] : 0;
            const std::int64_t gn = slot_tile(gemm_slot(gelu, wn, ni)) * kTileRows + col;
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rl = wm * 64 + mi * 16 + 4 * L + r;
                    const int P = acc_i[mi][ni][r];
                    int Pp;
                    if constexpr (BITS == 8) Pp = a.is_static ? P : P - meta.a_z[gi][rl] * cs;
                    else Pp = P - zw * meta.a_q[gi][rl];
                    if (a.dump) {
                        const std::int64_t gm = m0 + rl;
                        if (gm < a.M && gn < a.N && b < a.groups) a.dump[(gm * a.N + gn) * a.groups + b] = Pp;
                    }
                    float t = s * static_cast<float>(Pp);
                    if (BITS != 8 && a.zero_mode == ZERO_FLOAT) t = t + zf * static_cast<float>(meta.a_q[gi][rl]);
                    acc_f[mi][ni][r] = a.is_static ? acc_f[mi][ni][r] + t : acc_f[mi][ni][r] + meta.a_s[gi][rl] * t;
                }
                acc_i[mi][ni] = v4i{0, 0, 0, 0};
            }
        }
    };

    for (std::int64_t kt = 0; kt < a.k_tiles; ++kt) {
        __syncthreads();
        // stage activations: GM rows x KT bytes
        for (int c = tid; c < GM * KT / 16; c += 256) {
            const int r = c / (KT / 16), o = (c % (KT / 16)) * 16;
            const uint4 v = *reinterpret_cast<const uint4*>(a.q + (m0 + r) * a.cols_p + kt * KT + o);
            *reinterpret_cast<uint4*>(lds_a + r * AS + o) = v;
        }
        // stage weights: 8 tiles x 1 KiB
        for (int c = tid; c < 8 * 64; c += 256) {
            const int t = c / 64, s = c % 64;
            const std::int64_t nt = slot_tile(t);
            uint4 v = make_uint4(0, 0, 0, 0);
            if (nt < a.n_tiles) v = *reinterpret_cast<const uint4*>(a.tiles + (nt * a.k_tiles + kt) * kTileBytes + 16 * s);
            *reinterpret_cast<uint4*>(lds_b + t * kTileBytes + 16 * s) = v;
        }
        // stage the metadata of the groups that close in this tile
        const int b0 = static_cast<int>(a.group >= KT ? kt / tiles_per_group : kt * gpt);
        const bool group_ends = a.group < KT || (kt + 1) % tiles_per_group == 0;
        if (group_ends) {
            for (int c = tid; c < gpt * GM; c += 256) {
                const int gi = c / GM, r = c % GM;
                const std::int64_t ab = (m0 + r) * a.groups_p + b0 + gi;
                meta.a_s[gi][r] = a.a_scale[ab];
                meta.a_q[gi][r] = a.a_sum[ab];
                if constexpr (BITS == 8) meta.a_z[gi][r] = a.a_zero[ab];
            }
            for (int c = tid; c < gpt * GN; c += 256) {
                const int gi = c / GN, r = c % GN;
                const std::int64_t nt = slot_tile(r / 16);
                float s = 0.F, zf = 0.F;
                int zw = sign_offset(BITS), cs = 0;
                if (nt < a.n_tiles) {
                    const int rr = r % 16;
                    const std::int64_t mi = (nt * a.groups_p + b0 + gi) * kTileRows + rr;
                    s = meta_load(static_cast<const ST*>(a.scales), mi);
                    if (BITS == 8) cs = a.code_sums[mi];
                    if (a.zero_mode == ZERO_POINT) zw = (a.zero_points[(mi - rr) / 2 + rr / 2] >> (4 * (rr & 1))) & 15;
                    if (a.zero_mode == ZERO_FLOAT)
                        zf = a.zero_half ? __half2float(static_cast<const __half*>(a.zeros)[mi]) : static_cast<const float*>(a.zeros)[mi];
                }
                meta.s[gi][r] = s;
                meta.zw[gi][r] = zw;
                if constexpr (BITS == 4) meta.zf[gi][r] = zf;
                if constexpr (BITS == 8) meta.cs[gi][r] = cs;
            }
        }
        __syncthreads();

        uint4 bslot[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            bslot[ni] = *reinterpret_cast<const uint4*>(lds_b + gemm_slot(gelu, wn, ni) * kTileBytes + 16 * lane);

#pragma unroll
        for (int j = 0; j < J; ++j) {
            int bo[4][4];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                if constexpr (J == 1) unpack_block<BITS, 0>(bslot[ni], bo[ni]);
                else if constexpr (J == 2) {
                    if (j == 0) unpack_block<BITS, 0>(bslot[ni], bo[ni]);
                    else unpack_block<BITS, 1>(bslot[ni], bo[ni]);
                } else {
                    if (j == 0) unpack_block<BITS, 0>(bslot[ni], bo[ni]);
                    else if (j == 1) unpack_block<BITS, 1>(bslot[ni], bo[ni]);
                    else if (j == 2) unpack_block<BITS, 2>(bslot[ni], bo[ni]);
                    else unpack_block<BITS, 3>(bslot[ni], bo[ni]);
                }
            }
            uint4 av[4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
                av[mi] = *reinterpret_cast<const uint4*>(lds_a + (wm * 64 + mi * 16 + col) * AS + 64 * j + 16 * L);
            if (a.group == 32) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi) {
                        const long aa = h == 0 ? static_cast<long>((static_cast<std::uint64_t>(av[mi].y) << 32) | av[mi].x)
                                               : static_cast<long>((static_cast<std::uint64_t>(av[mi].w) << 32) | av[mi].z);
#pragma unroll
                        for (int ni = 0; ni < 4; ++ni) {
                            const long bb = static_cast<long>(
                                (static_cast<std::uint64_t>(static_cast<std::uint32_t>(bo[ni][2 * h + 1])) << 32) |
                                static_cast<std::uint32_t>(bo[ni][2 * h]));
                            acc_i[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aa, bb, acc_i[mi][ni], 0, 0, 0);
                        }
                    }
                    epilogue(2 * j + h, b0 + 2 * j + h);
                }
            } else {
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) {
                    const v4i aa = v4i{static_cast<int>(av[mi].x), static_cast<int>(av[mi].y), static_cast<int>(av[mi].z),
                                       static_cast<int>(av[mi].w)};
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni) {
                        const v4i bb = v4i{bo[ni][0], bo[ni][1], bo[ni][2], bo[ni][3]};
                        acc_i[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa, bb, acc_i[mi][ni], 0, 0, 0);
                    }
                }
                if (a.group < KT && ((j + 1) * 64) % a.group == 0) {
                    const int gi = (j * 64) / a.group;
                    epilogue(gi, b0 + gi);
                }
            }
        }
        if (a.group >= KT && group_ends) epilogue(0, b0);
    }

    // store
    if (!gelu) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const std::int64_t gn = slot_tile(gemm_slot(false, wn, ni)) * kTileRows + col;
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const std::int64_t gm = m0 + wm * 64 + mi * 16 + 4 * L + r;
                    float v = acc_f[mi][ni][r];
                    if (a.is_static) v = v * a.input_scale;
                    v = calibrate_output(v, a.output_scale);
                    if (gm < a.M && gn < a.N) a.y[gm * a.N + gn] = v;
                }
        }
    } else {
        const std::int64_t half_n = a.N / 2;
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const std::int64_t gi_tile = nb * 4 + 2 * wn + ni;
            const std::int64_t i = gi_tile * kTileRows + col;
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const std::int64_t gm = m0 + wm * 64 + mi * 16 + 4 * L + r;
                    float g = acc_f[mi][ni][r], up = acc_f[mi][ni + 2][r];
                    if (a.is_static) {
                        g = g * a.input_scale;
                        up = up * a.input_scale;
                    }
                    g = calibrate_output(g, a.output_scale);
                    up = calibrate_output(up, a.output_scale);
                    if (gm < a.M && gi_tile < half_tiles && i < half_n) a.y[gm * half_n + i] = gelu_tanh(g) * up;
                }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Row-major (Kidi layout) integer path for group sizes the tiles cannot carry: one thread per output, exact int32
// per group, epilogue in the oracle's order.
template <int BITS, typename ST>
__device__ float rowmajor_output(const LinearArgs& a, std::int64_t m, std::int64_t n) {
    const std::int64_t row_bytes = a.K / (8 / BITS);
    const std::uint8_t* row = a.tiles + n * row_bytes;
    float acc = 0.F;
    for (int b = 0; b < a.groups; ++b) {
        int P = 0, C = 0;
        for (int c = 0; c < a.group; ++c) {
            const std::int64_t k = static_cast<std::int64_t>(b) * a.group + c;
            const int w = kidi_code(row, BITS, k);
            P += static_cast<int>(a.q[m * a.K + k]) * w;
            C += w;
        }
        const std::int64_t meta = n * a.groups + b, ab = m * a.groups + b;
        const float s = meta_load(static_cast<const ST*>(a.scales), meta);
        int Pp = P;
        if (BITS == 8 && !a.is_static) Pp = P - a.a_zero[ab] * C;
        if (a.zero_mode == ZERO_POINT) Pp = P + (8 - static_cast<int>(a.zero_points[meta])) * a.a_sum[ab];  // sum q*(u - zp)
        if (a.dump) a.dump[(m * a.N + n) * a.groups + b] = Pp;
        float t = s * static_cast<float>(Pp);
        if (a.zero_mode == ZERO_FLOAT) {
            const float z = a.zero_half ? __half2float(static_cast<const __half*>(a.zeros)[meta]) : static_cast<const float*>(a.zeros)[meta];
            t = t + z * static_cast<float>(a.a_sum[ab]);
        }
        acc = a.is_static ? acc + t : acc + a.a_scale[ab] * t;
    }
    if (a.is_static) acc = acc * a.input_scale;
    return calibrate_output(acc, a.output_scale);
}

// One thread per output; with a.gelu one thread per gated output (gate row i and up row i + N/2).
template <int BITS, typename ST>
__global__ __launch_bounds__(256) void rowmajor_kernel(LinearArgs a) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::int64_t cols = a.gelu ? a.N / 2 : a.N;
    if (id >= a.M * cols) return;
    const std::int64_t m = id / cols, n = id % cols;
    if (a.gelu) a.y[id] = gelu_tanh(rowmajor_output<BITS, ST>(a, m, n)) * rowmajor_output<BITS, ST>(a, m, n + cols);
    else a.y[id] = rowmajor_output<BITS, ST>(a, m, n);
}

template <int BITS, typename ST>
__device__ float portable_output(const LinearArgs& a, int tiled, std::int64_t m, std::int64_t n) {
    const std::int64_t row_bytes = a.K / (8 / BITS);
    float acc = 0.F;
    for (std::int64_t k = 0; k < a.K; ++k) {
        const std::int64_t b = k / a.group;
        int c;
        std::int64_t meta;
        if (tiled) {
            const CodePos p = code_position(BITS, a.k_tiles, n, k);
            const int raw = (a.tiles[p.byte] >> p.shift) & ((1 << BITS) - 1);
            c = BITS == 8 ? static_cast<std::int8_t>(a.tiles[p.byte]) : raw - sign_offset(BITS);
            meta = (n / kTileRows * a.groups_p + b) * kTileRows + n % kTileRows;
        } else {
            c = kidi_code(a.tiles + n * row_bytes, BITS, k);
            meta = n * a.groups + b;
        }
        const float s = meta_load(static_cast<const ST*>(a.scales), meta);
        float w = static_cast<float>(c) * s;
        if (a.parity) {
            // runtime::parity::packed_linear (parity_math.cpp:247-277): x on the calibration grid, w = c * s, one
            // fused multiply-add per column in order
            const float xv = clampf(__builtin_rintf(load_act(a.x, a.x_type, m * a.K + k) / a.input_scale), -128.F, 127.F) *
                             a.input_scale;
            acc = __builtin_fmaf(xv, w, acc);
            continue;
        }
        if (a.zero_mode == ZERO_POINT) {
            int zp;
            if (tiled) zp = (a.zero_points[(meta - n % kTileRows) / 2 + (n % kTileRows) / 2] >> (4 * (n & 1))) & 15;
            else zp = a.zero_points[meta];
            w = w + (8.0F - static_cast<float>(zp)) * s;
        } else if (a.zero_mode == ZERO_FLOAT) {
            w = w + (a.zero_half ? __half2float(static_cast<const __half*>(a.zeros)[meta]) : static_cast<const float*>(a.zeros)[meta]);
        }
        float xv = load_act(a.x, a.x_type, m * a.K + k);
        if (a.input_scale > 0.F) xv = clampf(__builtin_rintf(xv / a.input_scale), -128.F, 127.F) * a.input_scale;
        acc = acc + xv * w;
    }
    return calibrate_output(acc, a.output_scale);
}

// Kidi's portable float path (PortablePackedLinearOp, operators.cpp:2639-2713): w = c*s (+ z), activations
// statically rounded when input_scale > 0, fp32 sum over k in order, output rounding. One thread per output; with
// a.gelu one thread per gated output (gate row i and up row i + N/2).
template <int BITS, typename ST>
__global__ __launch_bounds__(256) void portable_kernel(LinearArgs a, int tiled) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::int64_t cols = a.gelu ? a.N / 2 : a.N;
    if (id >= a.M * cols) return;
    const std::int64_t m = id / cols, n = id % cols;
    if (a.gelu) a.y[id] = gelu_tanh(portable_output<BITS, ST>(a, tiled, m, n)) * portable_output<BITS, ST>(a, tiled, m, n + cols);
    else a.y[id] = portable_output<BITS, ST>(a, tiled, m, n);
}

// GELU-tanh gating over a [M, 2I] buffer (used after the GEMM / row-major / portable kernels).
__global__ __launch_bounds__(256) void gelu_gate_kernel(const float* in, std::int64_t M, std::int64_t I, float* out) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= M * I) return;
    const std::int64_t m = id / I, i = id % I;
    out[id] = gelu_tanh(in[m * 2 * I + i]) * in[m * 2 * I + I + i];
}

// SiLU gating h = g / (1 + exp(-g)) * up (Context::silu_multiply, ops/context.cpp:964-969; eager_test.cpp:176-179)
__global__ __launch_bounds__(256) void silu_gate_kernel(const float* in, std::int64_t M, std::int64_t I, float* out) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= M * I) return;
    const std::int64_t m = id / I, i = id % I;
    const float g = in[m * 2 * I + i];
    out[id] = g / (1.F + expf(-g)) * in[m * 2 * I + I + i];
}

// act(gate) * value over two matching F32 buffers: Context::gelu_multiply / silu_multiply (ops/context.cpp:944-957),
// the slice form of the two gate kernels above (layers/gemma4.cpp:213-225), with their expressions, so
// gated_multiply(g, u) equals the gate kernels on [g | u] bit for bit. Four elements per thread (16-byte accesses
// when the buffers allow).
template <bool SILU>
__device__ __forceinline__ float gated(float g, float u) {
    if constexpr (SILU) return g / (1.F + expf(-g)) * u;
    return gelu_tanh(g) * u;
}
template <bool SILU, bool VEC>
__global__ __launch_bounds__(256) void gated_multiply_kernel(const float* gate, const float* value, std::int64_t n, float* out) {
    const std::int64_t i0 = (static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
    if (i0 >= n) return;
    if (VEC && i0 + 4 <= n) {
        const float4 g = *reinterpret_cast<const float4*>(gate + i0), u = *reinterpret_cast<const float4*>(value + i0);
        *reinterpret_cast<float4*>(out + i0) = make_float4(gated<SILU>(g.x, u.x), gated<SILU>(g.y, u.y), gated<SILU>(g.z, u.z),
                                                          gated<SILU>(g.w, u.w));
        return;
    }
    for (std::int64_t i = i0; i < n && i < i0 + 4; ++i) out[i] = gated<SILU>(gate[i], value[i]);
}

__global__ __launch_bounds__(256) void unpermute_kernel(const std::int8_t* q, std::int64_t M, std::int64_t K,
                                                        std::int64_t cols_p, std::int8_t* codes) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= M * K) return;
    const std::int64_t m = id / K, k = id % K;
    codes[id] = q[m * cols_p + act_position(k)];
}

__global__ __launch_bounds__(256) void block_stats_kernel(const float* s_in, const std::int32_t* q_in, const std::int32_t* z_in,
                                                          std::int64_t M, int groups, int groups_p, float* s,
                                                          std::int32_t* q, std::int32_t* z) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= M * groups) return;
    const std::int64_t m = id / groups, b = id % groups;
    if (s) s[id] = s_in[m * groups_p + b];
    if (q) q[id] = q_in[m * groups_p + b];
    if (z) z[id] = z_in[m * groups_p + b];
}

int pow2_floor(int v) {
    int p = 1;
    while (p * 2 <= v) p *= 2;
    return p;
}


template <int BITS, typename ST>
hipError_t launch_gemv_bits(const LinearCall& c, LinearArgs a, hipStream_t stream) {
    const Weight& w = *c.w;
    constexpr int KT = 512 / BITS;
    a.tiles_per_unit = w.geo.group >= KT ? w.geo.group / KT : 1;
    a.units = static_cast<int>(w.geo.k_tiles / a.tiles_per_unit);
    const std::int64_t blocks = c.gelu_gate ? w.geo.n_tiles / 2 : w.geo.n_tiles;
    int waves = static_cast<int>(std::max<std::int64_t>(1, 4096 / std::max<std::int64_t>(1, blocks)));
    waves = std::min(waves, 16);
    waves = std::min(waves, a.units);
    waves = pow2_floor(std::max(1, waves));
    const dim3 grid(static_cast<unsigned>(blocks)), block(64 * waves);
#define KQ_GEMV(MM, UU)                                                                                        \
    do {                                                                                                       \
        if (c.gelu_gate) hipLaunchKernelGGL((gemv_gelu_kernel<BITS, MM, ST, UU>), grid, block, 0, stream, a);  \
        else hipLaunchKernelGGL((gemv_kernel<BITS, MM, ST, UU>), grid, block, 0, stream, a);                   \
    } while (0)
    switch (c.M) {
    case 1: KQ_GEMV(1, 4); break;
    case 2: KQ_GEMV(2, 2); break;
    case 3: KQ_GEMV(3, 1); break;
    case 4: KQ_GEMV(4, 1); break;
    default: KQ_GEMV(8, 1); break;
    }
#undef KQ_GEMV
    return hipGetLastError();
}

template <int BITS, typename ST>
hipError_t launch_tiled(const LinearCall& c, hipStream_t stream) {
    LinearArgs a = make_linear_args(c);
    if (c.M <= 8) return launch_gemv_bits<BITS, ST>(c, a, stream);
    const std::int64_t m_blocks = (c.M + GM - 1) / GM;
    const std::int64_t n_blocks = c.gelu_gate ? (c.w->geo.n_tiles / 2 + 3) / 4 : (c.w->geo.n_tiles + 7) / 8;
    hipLaunchKernelGGL((gemm_kernel<BITS, ST>), dim3(static_cast<unsigned>(m_blocks * n_blocks)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int BITS, typename ST>
hipError_t launch_rowmajor(const LinearCall& c, hipStream_t stream) {
    LinearArgs a = make_linear_args(c);
    const std::int64_t total = c.M * (c.gelu_gate ? c.w->geo.rows / 2 : c.w->geo.rows);
    hipLaunchKernelGGL((rowmajor_kernel<BITS, ST>), dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int BITS, typename ST>
hipError_t launch_portable(const LinearCall& c, hipStream_t stream) {
    LinearArgs a = make_linear_args(c);
    const std::int64_t total = c.M * (c.gelu_gate ? c.w->geo.rows / 2 : c.w->geo.rows);
    hipLaunchKernelGGL((portable_kernel<BITS, ST>), dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, a,
                       c.w->tiled ? 1 : 0);
    return hipGetLastError();
}

template <typename ST>
hipError_t dispatch_bits(const LinearCall& c, hipStream_t stream, int kind) {
    switch (c.w->geo.bits) {
    case 2: return kind == 0 ? launch_tiled<2, ST>(c, stream) : kind == 1 ? launch_rowmajor<2, ST>(c, stream) : launch_portable<2, ST>(c, stream);
    case 4: return kind == 0 ? launch_tiled<4, ST>(c, stream) : kind == 1 ? launch_rowmajor<4, ST>(c, stream) : launch_portable<4, ST>(c, stream);
    default: return kind == 0 ? launch_tiled<8, ST>(c, stream) : kind == 1 ? launch_rowmajor<8, ST>(c, stream) : launch_portable<8, ST>(c, stream);
    }
}

}  // namespace

hipError_t launch_quantize(const LinearCall& c, hipStream_t stream) {
    const Weight& w = *c.w;
    if (c.path == PATH_PORTABLE) return hipSuccess;
    QuantArgs q{};
    q.x = c.x;
    q.x_type = c.x_type;
    q.M = c.M;
    q.K = w.geo.cols;
    q.group = w.geo.group;
    q.input_scale = c.input_scale;
    q.q = c.act.q;
    q.scale = c.act.scale;
    q.sum = c.act.sum;
    q.zero = c.act.zero;
    const int mode = c.path == PATH_SYMMETRIC ? 2 : (w.geo.bits == 8 ? 1 : 0);
    if (w.tiled) {
        q.cols_p = w.geo.cols_p;
        q.rows_p = c.act.rows_p;
        q.groups_p = static_cast<int>(w.geo.groups_p);
        const int chunks = w.geo.group / 8;
        q.lanes = chunks >= 64 ? 64 : pow2_floor(chunks);
        if (q.lanes != chunks && chunks < 64) q.lanes = 64;  // non power-of-two groups loop over chunks
        q.permuted = 1;
        const std::int64_t groups = q.rows_p * q.groups_p;
        const std::int64_t waves = (groups + (64 / q.lanes) - 1) / (64 / q.lanes);
        const dim3 grid(static_cast<unsigned>((waves + 3) / 4)), block(256);
        if (mode == 0) hipLaunchKernelGGL(quantize_kernel<0>, grid, block, 0, stream, q);
        else if (mode == 1) hipLaunchKernelGGL(quantize_kernel<1>, grid, block, 0, stream, q);
        else hipLaunchKernelGGL(quantize_kernel<2>, grid, block, 0, stream, q);
    } else {
        q.cols_p = w.geo.cols;
        q.rows_p = c.M;
        q.groups_p = static_cast<int>(w.geo.cols / w.geo.group);
        q.permuted = 0;
        const std::int64_t total = c.M * q.groups_p;
        const dim3 grid(static_cast<unsigned>((total + 255) / 256)), block(256);
        if (mode == 0) hipLaunchKernelGGL(quantize_rowmajor_kernel<0>, grid, block, 0, stream, q);
        else if (mode == 1) hipLaunchKernelGGL(quantize_rowmajor_kernel<1>, grid, block, 0, stream, q);
        else hipLaunchKernelGGL(quantize_rowmajor_kernel<2>, grid, block, 0, stream, q);
    }
    return hipGetLastError();
}

hipError_t launch_linear(const LinearCall& c, hipStream_t stream) {
    const int kind = c.path == PATH_PORTABLE ? 2 : (c.w->tiled ? 0 : 1);
    if (c.w->scale_type == META_F16) return dispatch_bits<__half>(c, stream, kind);
    return dispatch_bits<float>(c, stream, kind);
}

hipError_t launch_gated_multiply(const float* gate, const float* value, std::int64_t n, bool silu, float* out, hipStream_t stream) {
    const bool vec = !((reinterpret_cast<std::uintptr_t>(gate) | reinterpret_cast<std::uintptr_t>(value) |
                        reinterpret_cast<std::uintptr_t>(out)) & 15u);
    const dim3 grid(static_cast<unsigned>((n + 1023) / 1024)), block(256);
    if (silu) {
        if (vec) hipLaunchKernelGGL((gated_multiply_kernel<true, true>), grid, block, 0, stream, gate, value, n, out);
        else hipLaunchKernelGGL((gated_multiply_kernel<true, false>), grid, block, 0, stream, gate, value, n, out);
    } else {
        if (vec) hipLaunchKernelGGL((gated_multiply_kernel<false, true>), grid, block, 0, stream, gate, value, n, out);
        else hipLaunchKernelGGL((gated_multiply_kernel<false, false>), grid, block, 0, stream, gate, value, n, out);
    }
    return hipGetLastError();
}

hipError_t launch_gelu_gate(const float* in, std::int64_t M, std::int64_t I, float* out, hipStream_t stream) {
    const std::int64_t total = M * I;
    hipLaunchKernelGGL(gelu_gate_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, in, M, I, out);
    return hipGetLastError();
}

hipError_t launch_silu_gate(const float* in, std::int64_t M, std::int64_t I, float* out, hipStream_t stream) {
    const std::int64_t total = M * I;
    hipLaunchKernelGGL(silu_gate_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, in, M, I, out);
    return hipGetLastError();
}

hipError_t launch_unpermute_codes(const Weight& w, const ActBuffers& act, std::int64_t M, std::int8_t* codes,
                                  hipStream_t stream) {
    const std::int64_t total = M * w.geo.cols;
    if (!w.tiled) return hipMemcpyAsync(codes, act.q, static_cast<std::size_t>(total), hipMemcpyDeviceToDevice, stream);
    hipLaunchKernelGGL(unpermute_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, act.q, M,
                       w.geo.cols, w.geo.cols_p, codes);
    return hipGetLastError();
}

hipError_t launch_copy_block_stats(const Weight& w, const ActBuffers& act, std::int64_t M, float* scales,
                                   std::int32_t* sums, std::int32_t* zero_points, hipStream_t stream) {
    const int groups = static_cast<int>(w.geo.cols / w.geo.group);
    const int groups_p = w.tiled ? static_cast<int>(w.geo.groups_p) : groups;
    const std::int64_t total = M * groups;
    hipLaunchKernelGGL(block_stats_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, act.scale,
                       act.sum, act.zero, M, groups, groups_p, scales, sums, zero_points);
    return hipGetLastError();
}

namespace dev {

LinearArgs make_linear_args(const LinearCall& c) {
    const Weight& w = *c.w;
    LinearArgs a{};
    a.x = c.x;
    a.x_type = c.x_type;
    a.tiles = w.tiles;
    a.scales = w.scales;
    a.zero_points = w.zero_points;
    a.zeros = w.zeros;
    a.code_sums = w.code_sums;
    a.q = c.act.q;
    a.a_scale = c.act.scale;
    a.a_sum = c.act.sum;
    a.a_zero = c.act.zero;
    a.y = c.y;
    a.dump = c.dump;
    a.M = c.M;
    a.N = w.geo.rows;
    a.K = w.geo.cols;
    a.cols_p = w.geo.cols_p;
    a.k_tiles = w.geo.k_tiles;
    a.n_tiles = w.geo.n_tiles;
    a.group = w.geo.group;
    a.groups_p = static_cast<int>(w.geo.groups_p);
    a.groups = static_cast<int>(w.geo.cols / w.geo.group);
    a.zero_mode = w.zero_mode;
    a.zero_half = w.zero_type == META_F16;
    a.is_static = c.path == PATH_SYMMETRIC;
    a.gelu = c.gelu_gate;
    a.parity = c.parity ? 1 : 0;
    a.input_scale = c.input_scale;
    a.output_scale = c.output_scale;
    a.dq_codes = c.dq_codes;
    a.dq_scales = c.dq_scales;
    a.dq_sums = c.dq_sums;
    a.dq_zeros = c.dq_zeros;
    return a;
}

}  // namespace dev

}  // namespace kq
