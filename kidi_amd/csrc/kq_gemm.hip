// Prefill projection (M > 16) of the MI355X quantized linear layer for 4-bit weights with g = 128 (symmetric or
// with zero points) and K a multiple of 512: an activation quantizer and an int8 MFMA GEMM.
//
// quantize_rows_kernel: one lane per 32 columns of a row, a lane quad per group (max |x| reduced with DPP); codes go
//   to [M_p][K] in the tiles' permuted order, block scales to [groups][M_p] (transposed so a GEMM stage copies one
//   contiguous 1 KiB row of them).
// gemm_i4_kernel: workgroup tile 256 (rows) x 128 (output columns = 8 weight row tiles), 8 waves of 64 x 64, one
//   128-column k-step (= one 4-bit tile = one group) per iteration, operands in LDS rings:
//     - activation codes: 32 direct-to-LDS copies of 1 KiB per step (buffer_load ... lds), lane addresses XOR-
//       swizzled by row so A-operand reads spread over the LDS banks;
//     - weights: packed tiles copied to LDS the same way; each wave unpacks one (two) of them to int8 with the zero
//       point folded in (u - zp per byte, SWAR) and stores both 64-column halves in B-operand order;
//     - MFMA: per 64-column half 4 A and 4 B reads, 16 v_mfma_i32_16x16x64_i8; the int32 accumulators hold the
//       exact per-group partials P' = sum q (u - zp);
//     - epilogue per group: acc += a_s[row] * s[col] * P' (calibrated: s * P', input_scale applied at the end).
// Numerics: BlockwiseLinear / SymmetricPackedLinear closed forms (runtime/ynn/operators.cpp:1118-1169,
// :1250-1308) with the zero point folded into the integer operand: w = (u - zp) * s = c * s + (8 - zp) * s.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "kq_device.hpp"
#include "kq_internal.hpp"

namespace kq {
namespace {

using namespace dev;

typedef __attribute__((address_space(3))) void lds_void;
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kBK = 128;  // columns per step (one group); a workgroup's 128 output columns are 8 row tiles
constexpr int kBBytes = 8 * 2 * 1024;   // unpacked weights per stage: [tile slot][64-column half][lane][16 B]
constexpr int kQuantRows = 256;         // activation rows are padded to this for every tile shape

// Workgroup tile: WM x 2 waves of 64 x 64 outputs; BM = 64 WM rows x 128 columns (one group) per k step. Every
// global operand reaches LDS through direct copies (buffer_load ... lds), so no loaded register waits on memory:
//   - activation codes, weight scales, activation scales: copied three steps ahead into a 3-slot ring;
//   - packed int4 weight tiles and zero points: copied four steps ahead into a 3-slot ring, unpacked to int8
//     (zero point folded in) LDS to LDS during the previous step into a 2-slot ring of B operands.
// One barrier per step, in the middle of it; before it, s_waitcnt vmcnt(copies of the previous step) leaves only
// those in flight.
template <int WM>
struct GemmShape {
    static constexpr int BM = 64 * WM, WAVES = 2 * WM, THREADS = 64 * WAVES;
    static constexpr int TPW = 8 / WAVES;                 // weight tiles each wave copies and unpacks per step
    static constexpr int A_BYTES = BM * kBK;              // activation codes per slot
    static constexpr int RAW_BYTES = 8 * kTileBytes;      // packed weight tiles per slot
    static constexpr int WS_OFF = 0, ZP_OFF = 512, AS_OFF = 768;  // inside a metadata slot
    static constexpr int META_BYTES = AS_OFF + BM * 4;
    static constexpr int A_RING = 0;
    static constexpr int RAW_RING = A_RING + 3 * A_BYTES;
    static constexpr int BQ_RING = RAW_RING + 3 * RAW_BYTES;
    static constexpr int META_RING = BQ_RING + 2 * kBBytes;
    static constexpr int SCRATCH = META_RING + 3 * META_BYTES;  // 256 bytes that idle copies write into
    static constexpr int LDS = SCRATCH + 256;
    static_assert(LDS <= 160 * 1024, "LDS budget");
};

// LDS reads and writes of the k loop are inline assembly with explicit lgkmcnt/vmcnt waits: the compiler cannot
// tell a read of one ring slot from the copies in flight into the others, and would wait for those copies before
// every read. Each wait ties the registers it guards, so no use can move above it.
__device__ __forceinline__ std::uint32_t lds_addr(void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>((lds_void*)p));
#else
    return static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>(p));
#endif
}
// (the host pass sees these bodies too; the asm is device-only)
#if defined(__HIP_DEVICE_COMPILE__)
#define KQ_ASM(...) asm volatile(__VA_ARGS__)
#else
#define KQ_ASM(...) (void)0
#endif
template <int OFF>
__device__ __forceinline__ v4i ds_read16(std::uint32_t addr) {
    v4i v = {0, 0, 0, 0};
    KQ_ASM("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ std::uint32_t ds_read4(std::uint32_t addr) {
    std::uint32_t v = 0;
    KQ_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ std::uint32_t ds_read2(std::uint32_t addr) {
    std::uint32_t v = 0;
    KQ_ASM("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ std::uint32_t ds_read1(std::uint32_t addr) {
    std::uint32_t v = 0;
    KQ_ASM("ds_read_u8 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ void ds_write16(std::uint32_t addr, v4u v) {
    KQ_ASM("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "n"(OFF));
}
template <typename T>
__device__ __forceinline__ void tie(T& x) {
    KQ_ASM("" : "+v"(x));
}
template <int N, typename... T>
__device__ __forceinline__ void lgkm_wait(T&... x) {
    KQ_ASM("s_waitcnt lgkmcnt(%0)" : : "n"(N));
    // the empty statements below make every guarded register an output of code after the wait
    (tie(x), ...);
}

constexpr int kRsrcWord3 = 0x00020000;
constexpr std::uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kRsrcWord3);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, std::uint32_t off) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
// Position of row m's block scale inside a [groups][M_p] row of the transposed scales: within each 64-row block,
// row 16 q + t is stored at 4 t + q, so the 4 rows 16 apart that one GEMM lane scales are adjacent.
__device__ __forceinline__ int scale_slot(int m) { return (m & ~63) | ((m & 15) << 2) | ((m >> 4) & 3); }

struct QRowArgs {
    const void* x;
    int x_f32;
    int M, M_p, K;
    float input_scale;
    std::int8_t* q;      // [M_p][K] permuted
    float* scale_t;      // [K/128][M_p]
    std::int32_t* sum_t; // [K/128][M_p] (optional)
    const float* ninv;   // NORM: per-row inverse RMS [M]
    const float* nw;     // NORM: norm weight [K]
};

// g = 128. One lane per 32 columns of a row: the pieces [16 a, 16 a + 16) and [32 + 16 a, 32 + 16 a + 16) of 64-column
// block b, lane unit j = 2 b + a. Their codes fill 32 contiguous bytes of the permuted row (column 32 h + 8 L + i of
// a 64-column block at 16 L + 8 h + i), and a group is one lane quad (2 DPP steps reduce it). Codes are packed with
// v_cvt_pk_u8_f32 on rint(x * inverse) + 128 (an integer in [1, 255]; calibrated codes clamped to [-128, 127]
// first), then the bias is flipped off per byte.
template <int QM, bool F32, bool NORM>
__global__ __launch_bounds__(256) void quantize_rows_kernel(QRowArgs a) {
    const int units = a.K / 32;  // lanes per row (a multiple of 16: rows never share a lane quad)
    const int t = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    const int m = t / units, j = t - m * units;
    if (m >= a.M_p) return;  // whole waves (M_p * units is a multiple of 64)
    const bool live = m < a.M;
    const int col0 = 64 * (j >> 1) + 16 * (j & 1);
    constexpr std::uint32_t ES = F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t xr = rsrc(a.x, static_cast<std::uint32_t>(a.M) * a.K * ES);
    const std::uint32_t e0 = (static_cast<std::uint32_t>(m) * a.K + col0) * ES;
    float v[32];  // v[0..15]: columns col0 + [0, 16); v[16..31]: col0 + 32 + [0, 16)
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const std::uint32_t off = live ? e0 + p * 32 * ES : kOob;
        if constexpr (F32) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 r = ld16(xr, off + 16 * i);
                v[16 * p + 4 * i] = __uint_as_float(r.x);
                v[16 * p + 4 * i + 1] = __uint_as_float(r.y);
                v[16 * p + 4 * i + 2] = __uint_as_float(r.z);
                v[16 * p + 4 * i + 3] = __uint_as_float(r.w);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 r = ld16(xr, off + 16 * i);
                const std::uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    v[16 * p + 8 * i + 2 * d] = __uint_as_float(w4[d] << 16);
                    v[16 * p + 8 * i + 2 * d + 1] = __uint_as_float(w4[d] & 0xFFFF0000u);
                }
            }
        }
    }
    if constexpr (NORM) {
        // fused RMS normalization: x * inv[m] * w[k] (the row's inverse RMS comes from rms_norm_kernel)
        const float inv = live ? a.ninv[m] : 0.F;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const float4* wp = reinterpret_cast<const float4*>(a.nw + col0 + 32 * p);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 w = wp[i];
                v[16 * p + 4 * i] = v[16 * p + 4 * i] * inv * w.x;
                v[16 * p + 4 * i + 1] = v[16 * p + 4 * i + 1] * inv * w.y;
                v[16 * p + 4 * i + 2] = v[16 * p + 4 * i + 2] * inv * w.z;
                v[16 * p + 4 * i + 3] = v[16 * p + 4 * i + 3] * inv * w.w;
            }
        }
    }
    float mx = 0.F, mn = 0.F;
    if constexpr (QM != QUANT_STATIC) {
#pragma unroll
        for (int i = 0; i < 32; ++i) quant_stat(QM, v[i], mx, mn);
        mx = fmaxf(mx, __int_as_float(dpp<0xB1>(__float_as_int(mx))));
        mx = fmaxf(mx, __int_as_float(dpp<0x4E>(__float_as_int(mx))));
    }
    const QuantBlock qb = quant_block(QM, mx, mn, a.input_scale, live);
    // output order: columns col0 + [0, 8), col0 + 32 + [0, 8), col0 + [8, 16), col0 + 32 + [8, 16)
    constexpr int kSrc[4] = {0, 16, 8, 24};
    std::uint32_t out[8];
    if constexpr (QM == QUANT_STATIC) {
        // calibrated: rint(x / input_scale) clamped to [-128, 127], + 128 packed as unsigned bytes, bias flipped off
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            std::uint32_t d = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float c = fminf(fmaxf(__builtin_rintf(v[kSrc[w >> 1] + 4 * (w & 1) + i] / a.input_scale), -128.F), 127.F);
                d = __builtin_amdgcn_cvt_pk_u8_f32(c + 128.F, i, d);
            }
            out[w] = d ^ 0x80808080u;
        }
    } else {
        // dynamic: |x * inverse| <= 127 (1 + 2^-24) rounds to at most 127 (no clamp). Adding 1.5 * 2^23 rounds
        // x * inverse to an integer (round to nearest even, as rint) held in the low mantissa bits, so the low byte
        // is the code in two's complement; v_perm gathers four of them.
        constexpr float kMagic = 12582912.F;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            std::uint32_t u[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) u[i] = __float_as_uint(v[kSrc[w >> 1] + 4 * (w & 1) + i] * qb.inverse + kMagic);
            const std::uint32_t lo = __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0400u), hi = __builtin_amdgcn_perm(u[3], u[2], 0x0c0c0400u);
            out[w] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
    }
    std::int8_t* dst = a.q + static_cast<std::int64_t>(m) * a.K + 64 * (j >> 1) + 32 * (j & 1);
    *reinterpret_cast<uint4*>(dst) = make_uint4(out[0], out[1], out[2], out[3]);
    *reinterpret_cast<uint4*>(dst + 16) = make_uint4(out[4], out[5], out[6], out[7]);
    // code sums (parity instrumentation only): from the packed bytes
    const bool sums = a.sum_t != nullptr;
    int q = 0;
    if (sums) {
#pragma unroll
        for (int w = 0; w < 8; ++w)
#pragma unroll
            for (int i = 0; i < 4; ++i) q += static_cast<std::int8_t>((out[w] >> (8 * i)) & 0xFFu);
        q += dpp<0xB1>(q);
        q += dpp<0x4E>(q);
    }
    if ((j & 3) == 0) {
        const std::int64_t o = static_cast<std::int64_t>(j >> 2) * a.M_p + scale_slot(m);
        a.scale_t[o] = qb.s;
        if (sums) a.sum_t[o] = q;
    }
}

// launch over M_p rows x K / 32 lanes
inline void launch_quantize_rows(const QRowArgs& q, bool calibrated, bool x_f32, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(static_cast<std::int64_t>(q.M_p) * (q.K / 32) / 256)), block(256);
#define KQ_QR(QM, F, NM) hipLaunchKernelGGL((quantize_rows_kernel<QM, F, NM>), grid, block, 0, stream, q)
#define KQ_QRN(QM, F) \
    if (q.ninv) KQ_QR(QM, F, true); \
    else KQ_QR(QM, F, false)
    if (calibrated) {
        if (x_f32) { KQ_QRN(dev::QUANT_STATIC, true); }
        else { KQ_QRN(dev::QUANT_STATIC, false); }
    } else {
        if (x_f32) { KQ_QRN(dev::QUANT_DYN_SYM, true); }
        else { KQ_QRN(dev::QUANT_DYN_SYM, false); }
    }
#undef KQ_QRN
#undef KQ_QR
}

struct GemmArgs {
    const std::int8_t* q;       // [M_p][K]
    const float* scale_t;       // [K/128][M_p]
    const std::uint8_t* tiles;
    const void* scales;         // [n_tiles][groups_p][16] F16|F32
    const std::uint8_t* zero_points;  // [n_tiles][groups_p][8], or null (symmetric: zero point 8)
    float* y;
    std::int32_t* dump;
    int M, M_p, N, K, k_tiles, n_tiles, groups_p, groups;
    int scale_half;
    float input_scale, output_scale;
    int m_blocks, n_blocks;
    int ksplit;          // K ranges per output tile (1, 2, 4 or 8)
    float* partial;      // ksplit > 1: fp32 partial tiles [ksplit][tiles][THREADS][64]
};

// Global row tile of LDS tile slot t (0..7) of column block nb, or n_tiles when out of range. GELU: slots 0-3 are
// gate tiles 4 nb + t, slots 4-7 the matching up tiles (gate rows [0, I), up rows [I, 2I)).
template <bool GELU>
__device__ __forceinline__ int slot_tile(const GemmArgs& a, int nb, int t) {
    if constexpr (GELU) {
        const int half = a.n_tiles >> 1;
        const int g = nb * 4 + (t & 3);
        return g < half ? (t < 4 ? g : half + g) : a.n_tiles;
    }
    const int nt = nb * 8 + t;
    return nt < a.n_tiles ? nt : a.n_tiles;
}
// LDS tile slot of wave column wn, subtile ni: plain 4 wn + ni; GELU 2 wn + ni (gate) / 4 + 2 wn + ni - 2 (up).
template <bool GELU>
__device__ __forceinline__ constexpr int wave_slot(int wn, int ni) {
    return GELU ? (ni < 2 ? 2 * wn + ni : 4 + 2 * wn + ni - 2) : 4 * wn + ni;
}

// Epilogue of one output tile: acc[mi][ni][r] is row m0 + 64 wm + 16 mi + 4 L + r, column 16 col_nt[ni] + nn;
// calibrated inputs scale by input_scale, calibrated outputs round to output_scale steps, GELU pairs gate and up.
template <int WM, bool GELU, int QM>
__device__ __forceinline__ void store_tile(const GemmArgs& a, const float (&acc)[4][4][4], int m0, const int (&col_nt)[4],
                                           int wm, int nn, int L, int only_mi = -1) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        if (only_mi >= 0 && mi != only_mi) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm * 64 + mi * 16 + 4 * L + r;
            if (row >= a.M) continue;
            if constexpr (GELU) {
                const int half_n = a.N >> 1;
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    const int i = col_nt[ni] * kTileRows + nn;
                    if (col_nt[ni] >= a.n_tiles || i >= half_n) continue;
                    float g = acc[mi][ni][r], up = acc[mi][ni + 2][r];
                    if (QM == QUANT_STATIC) {
                        g = g * a.input_scale;
                        up = up * a.input_scale;
                    }
                    g = calibrate_output(g, a.output_scale);
                    up = calibrate_output(up, a.output_scale);
                    a.y[static_cast<std::int64_t>(row) * half_n + i] = gelu_tanh(g) * up;
                }
            } else {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const int col = col_nt[ni] * kTileRows + nn;
                    if (col_nt[ni] >= a.n_tiles || col >= a.N) continue;
                    float v = acc[mi][ni][r];
                    if (QM == QUANT_STATIC) v = v * a.input_scale;
                    a.y[static_cast<std::int64_t>(row) * a.N + col] = calibrate_output(v, a.output_scale);
                }
            }
        }
    }
}

template <int WM, bool GELU, int QM, bool ZP, bool SH, bool DBG>
__global__ __launch_bounds__(GemmShape<WM>::THREADS) void gemm_i4_kernel(GemmArgs a) {
    using S = GemmShape<WM>;
    extern __shared__ __attribute__((aligned(16))) std::uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int nn = lane & 15, L = lane >> 4;
    const std::uint32_t lds0 = lds_addr(lds);

    // workgroup -> (row block, column block): consecutive workgroups go to different XCDs, so give each XCD a
    // contiguous range (its column blocks x all row blocks share its L2)
    const int tiles = a.m_blocks * a.n_blocks;
    const int total = tiles * a.ksplit;
    int bid = blockIdx.x;
    if (total % 8 == 0) bid = (bid % 8) * (total / 8) + bid / 8;
    const int ks = bid / tiles, tile = bid % tiles;  // K range ks of output tile `tile`
    const int mb = tile % a.m_blocks, nb = tile / a.m_blocks;
    const int m0 = mb * S::BM;
    const int nk = a.k_tiles / a.ksplit, kofs = ks * nk, kend = kofs + nk;  // groups [kofs, kend)

    // activation panel of this workgroup: rows [m0, m0 + BM) x K (rows are padded to a multiple of 256)
    const __amdgpu_buffer_rsrc_t ares = rsrc(a.q + static_cast<std::int64_t>(m0) * a.K, static_cast<std::uint32_t>(S::BM) * a.K);
    // packed weight tiles of the wave's slots (uniform per wave)
    int st_nt[S::TPW];
    __amdgpu_buffer_rsrc_t wres[S::TPW];
#pragma unroll
    for (int u = 0; u < S::TPW; ++u) {
        st_nt[u] = slot_tile<GELU>(a, nb, wave * S::TPW + u);
        const bool live = st_nt[u] < a.n_tiles;
        wres[u] = rsrc(a.tiles + static_cast<std::int64_t>(live ? st_nt[u] : 0) * a.k_tiles * kTileBytes,
                       live ? static_cast<std::uint32_t>(a.k_tiles * kTileBytes) : 0u);
    }
    // the wave's 4 output column tiles (uniform)
    int col_nt[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) col_nt[ni] = slot_tile<GELU>(a, nb, wave_slot<GELU>(wn, ni));
    // Metadata copies (4-byte lanes), META_N per wave, by role r = META_N wave + i: r = 0 the weight scales of the 8
    // tile slots (F16: all 8, lane l -> slot l / 8; F32: slots 0-3, lane l -> slot l / 16), r = 1 their zero points
    // (lane l < 16 -> slot l / 2), r = 2 .. WM + 1 the activation scales of rows [64 (r - 2), +64), r = WM + 2 (F32
    // only) the weight scales of slots 4-7; other roles copy zeros into the scratch area. Lane source byte:
    // base + step * k; out-of-range lanes read zeros.
    constexpr int META_N = (2 + WM + (SH ? 0 : 1) <= S::WAVES) ? 1 : 2;
    const std::uint32_t meta_n = static_cast<std::uint32_t>(a.n_tiles * a.groups_p * kTileRows);
    __amdgpu_buffer_rsrc_t mres[META_N];
    std::uint32_t meta_base[META_N], meta_step[META_N];
    int meta_dst[META_N];  // byte offset inside a metadata slot; -1: the scratch area
    bool meta_lead[META_N];  // zero points travel with the packed tiles (four steps ahead, the rest three)
#pragma unroll
    for (int i = 0; i < META_N; ++i) {
        const int role = wave * META_N + i;
        meta_base[i] = kOob;
        meta_step[i] = 0;
        meta_dst[i] = -1;
        meta_lead[i] = role == 1;
        mres[i] = rsrc(a.q, 0u);
        if (role == 0 || (!SH && role == WM + 2)) {
            constexpr int es = SH ? 2 : 4, lanes_per_slot = 16 * es / 4;
            const int t = (role == 0 ? 0 : 4) + lane / lanes_per_slot;
            const int nt = slot_tile<GELU>(a, nb, t);
            mres[i] = rsrc(a.scales, meta_n * es);
            meta_step[i] = kTileRows * es;
            if (nt < a.n_tiles) meta_base[i] = static_cast<std::uint32_t>(nt * a.groups_p) * kTileRows * es + (lane % lanes_per_slot) * 4;
            meta_dst[i] = S::WS_OFF + (role == 0 ? 0 : 256);
        } else if (role == 1) {
            const int nt = lane < 16 ? slot_tile<GELU>(a, nb, lane / 2) : a.n_tiles;
            mres[i] = rsrc(a.zero_points, ZP ? meta_n / 2 : 0u);
            meta_step[i] = 8;
            if (ZP && nt < a.n_tiles) meta_base[i] = static_cast<std::uint32_t>(nt * a.groups_p) * 8 + (lane % 2) * 4;
            meta_dst[i] = S::ZP_OFF;
        } else if (role < 2 + WM) {  // rows in the permuted order of scale_t
            mres[i] = rsrc(a.scale_t, static_cast<std::uint32_t>(a.groups_p) * a.M_p * 4);
            meta_step[i] = static_cast<std::uint32_t>(a.M_p) * 4;
            if (QM != QUANT_STATIC) meta_base[i] = static_cast<std::uint32_t>(m0 + 64 * (role - 2) + lane) * 4;
            meta_dst[i] = S::AS_OFF + 256 * (role - 2);
        }
    }

    // Copies of one step: activation codes of step ka into A slot ka % 3, packed tiles of step kb into raw slot
    // kb % 3, and this wave's metadata (step kb for zero points, else ka). The slot indices use the unclamped
    // step numbers; clamped steps copy the last group again into slots nobody reads.
    // Copy offsets: the lane part goes in the VGPR offset (computed once), the step part in the SGPR offset, so a
    // copy costs no vector instruction. Out-of-range lanes carry kOob in the VGPR part (their sum stays >= 2^31,
    // beyond every buffer); every other lane's sum is in range.
    // LDS byte 1024 i + 16 l of an A slot is row r = 8 i + l / 8, 16-byte chunk c' = l % 8, which holds global chunk
    // c = c' ^ (r & 7); i = 4 wave + part
    std::uint32_t a_voff[4];
#pragma unroll
    for (int part = 0; part < 4; ++part) {
        const int r = (wave * 4 + part) * 8 + (lane >> 3);
        a_voff[part] = static_cast<std::uint32_t>(r) * a.K + ((lane & 7) ^ (r & 7)) * 16;
    }
    auto issue_a = [&](int ka, int sa, int part) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lds_void*)(lds + S::A_RING + sa * S::A_BYTES + (wave * 4 + part) * 1024), 16,
                                                 a_voff[part], ka * kBK, 0, 0);
    };
    // (resources are copied out of their arrays: an array element passed to the builtin directly makes the host
    // pass drop the kernel's launch stub)
    auto issue_raw = [&](int kb, int sb) {
#pragma unroll
        for (int u = 0; u < S::TPW; ++u) {
            const __amdgpu_buffer_rsrc_t wr = wres[u];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(lds + S::RAW_RING + sb * S::RAW_BYTES + (wave * S::TPW + u) * kTileBytes),
                                                     16, static_cast<std::uint32_t>(lane * 16), kb * kTileBytes, 0, 0);
        }
    };
    // (ka < 0: only the zero points are copied, the other roles copy zeros into the scratch area)
    auto issue_meta = [&](int ka, int sa, int kb, int sb) {
#pragma unroll
        for (int i = 0; i < META_N; ++i) {
            const int km = meta_lead[i] ? kb : ka, sm = meta_lead[i] ? sb : sa;
            const bool idle = meta_dst[i] < 0 || km < 0;
            std::uint8_t* mdst = idle ? lds + S::SCRATCH : lds + S::META_RING + sm * S::META_BYTES + meta_dst[i];
            const __amdgpu_buffer_rsrc_t mr = mres[i];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(mr, (lds_void*)mdst, 4, km < 0 ? kOob : meta_base[i],
                                                     km < 0 ? 0u : meta_step[i] * static_cast<std::uint32_t>(km), 0, 0);
        }
    };
    // all copies of one step: activation codes of step ka into A slot sa, packed tiles of step kb into raw slot sb,
    // this wave's metadata (step kb for zero points, else ka)
    auto issue = [&](int ka, int sa, int kb, int sb) {
#pragma unroll
        for (int part = 0; part < 4; ++part) issue_a(ka, sa, part);
        issue_raw(kb, sb);
        issue_meta(ka, sa, kb, sb);
    };
    constexpr int kStepLoads = 4 + S::TPW + META_N;
    constexpr int kStepWait = (kStepLoads & 15) | (7 << 4) | ((kStepLoads >> 4) << 14);  // vmcnt(n) lgkmcnt(0)

    // Unpack the packed tiles of a step (raw slot sr, zero points in meta slot sm) into B slot sq: int8 with the
    // zero point folded in, byte = ((u | 0x80) - zp) ^ 0x80 = u - zp, in B-operand order [slot][half][lane][16 B].
    const std::uint32_t raw_lane = lds0 + S::RAW_RING + wave * S::TPW * kTileBytes + lane * 16;
    const std::uint32_t zp_lane = lds0 + S::META_RING + S::ZP_OFF + wave * S::TPW * 8 + (nn >> 1);
    const std::uint32_t bq_lane = lds0 + S::BQ_RING + wave * S::TPW * 2048 + lane * 16;
    struct Raw {
        v4i w[2];
        std::uint32_t zp[2];
    };
    auto unpack_read = [&](int sr, int sm) {
        Raw r;
        r.zp[0] = r.zp[1] = 8;
        r.w[0] = ds_read16<0>(raw_lane + sr * S::RAW_BYTES);
        if constexpr (S::TPW == 2) r.w[1] = ds_read16<kTileBytes>(raw_lane + sr * S::RAW_BYTES);
        if constexpr (ZP) {
            r.zp[0] = ds_read1<0>(zp_lane + sm * S::META_BYTES);
            if constexpr (S::TPW == 2) r.zp[1] = ds_read1<8>(zp_lane + sm * S::META_BYTES);
        }
        return r;
    };
    auto unpack_write = [&](Raw& r, int sq) {
        if constexpr (S::TPW == 1) lgkm_wait<0>(r.w[0], r.zp[0]);
        else lgkm_wait<0>(r.w[0], r.w[1], r.zp[0], r.zp[1]);
#pragma unroll
        for (int u = 0; u < S::TPW; ++u) {
            const std::uint32_t z = ZP ? ((r.zp[u] >> (4 * (nn & 1))) & 15u) : 8u;
            const std::uint32_t zz = __builtin_amdgcn_perm(0u, z, 0u);  // z in every byte (v_perm, not a multiply)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const std::uint32_t d0 = static_cast<std::uint32_t>(r.w[u][2 * j]), d1 = static_cast<std::uint32_t>(r.w[u][2 * j + 1]);
                v4u o;
                o.x = (((d0 & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                o.y = ((((d0 >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                o.z = (((d1 & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                o.w = ((((d1 >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zz) ^ 0x80808080u;
                const std::uint32_t dst = bq_lane + sq * kBBytes;
                if (u == 0 && j == 0) ds_write16<0>(dst, o);
                if (u == 0 && j == 1) ds_write16<1024>(dst, o);
                if (u == 1 && j == 0) ds_write16<2048>(dst, o);
                if (u == 1 && j == 1) ds_write16<3072>(dst, o);
            }
        }
    };
    auto unpack = [&](int sr, int sm, int sq) {
        Raw r = unpack_read(sr, sm);
        unpack_write(r, sq);
    };

    float acc[4][4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mi][ni][r] = 0.F;

    // Step schedule: one barrier per step, between blocks 7 and 8 (blocks are 16 x 16 output blocks, mi-major).
    //   - Step kt's operand registers are read during step kt - 1, each right after its last use there: metadata and
    //     A rows 0-1 after the barrier, A row 2 after block 12, B columns 0-2 after blocks 13-15, B column 3 and A
    //     row 3 last. By block 4 of step kt every operand of the step is in registers.
    //   - Blocks 4-6 unpack step kt + 1's packed tiles into B slot (kt + 1) % 2 (free since the previous barrier).
    //   - The barrier (after s_waitcnt vmcnt(copies of step kt - 1) lgkmcnt(0)) ends every read of step kt's A and
    //     metadata slots and of step kt + 1's raw slot, and publishes B slot (kt + 1) % 2. Blocks 8-13 then copy
    //     step kt + 3's activation codes and metadata into the slots of step kt, and step kt + 4's packed tiles and
    //     zero points into the raw / zero-point slots unpacked at blocks 4-6.
    // Ring slots are step - kofs modulo 3 (A, raw, metadata) and modulo 2 (B). Copies past the K range repeat the
    // range's last group into slots nobody reads.
    auto clamp_k = [&](int k) { return k < kend ? k : kend - 1; };
    {
        issue(kofs, 0, kofs, 0);
        issue(clamp_k(kofs + 1), 1, clamp_k(kofs + 1), 1);
        issue(clamp_k(kofs + 2), 2, clamp_k(kofs + 2), 2);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        unpack(0, 0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // packed tiles and zero points of step kofs + 3 into the slots step kofs used
        issue_raw(clamp_k(kofs + 3), 0);
        issue_meta(-1, 0, clamp_k(kofs + 3), 0);
    }

    // per-lane operand addresses (add the slot base per step)
    const int arow = wm * 64 + nn;  // A row of subtile 0 read by this lane
    const std::uint32_t a_lane0 = lds0 + S::A_RING + arow * kBK + ((L ^ (arow & 7)) * 16);
    const std::uint32_t a_lane1 = lds0 + S::A_RING + arow * kBK + (((4 + L) ^ (arow & 7)) * 16);
    // B operands of the wave's subtiles start at slot wave_slot(wn, 0) (plain 4 wn; GELU 2 wn: gate 2 wn, 2 wn + 1
    // and up 4 + 2 wn, 5 + 2 wn)
    const std::uint32_t b_lane = lds0 + S::BQ_RING + wave_slot<GELU>(wn, 0) * 2048 + lane * 16;
    constexpr int kWsStride = SH ? 32 : 64;  // bytes of one slot's 16 weight scales
    const std::uint32_t ws_lane = lds0 + S::META_RING + S::WS_OFF + wave_slot<GELU>(wn, 0) * kWsStride + nn * (SH ? 2 : 4);
    // activation scales of rows srow + 16 mi, mi = 0..3, srow = wm * 64 + t, t = 4 L + (lane & 3): adjacent in the
    // permuted order (row 16 q + t of a 64-row block at 4 t + q)
    const std::uint32_t as_lane = lds0 + S::META_RING + S::AS_OFF + (wm * 64 + 4 * (4 * L + (lane & 3))) * 4;
    const v4i zero = {0, 0, 0, 0};
#define KQ_BSLOT(ni) (GELU ? ((ni) < 2 ? (ni) : 2 + (ni)) : (ni))

    // operand registers of one step, read in this order: svr[0..3], asr, A0, A1 | A2 | B0 | B1 | B2 | B3, A3
    std::uint32_t svr[4];
    v4i asr = zero;
    v4i A[4][2], B[4][2];
    auto read_meta = [&](std::uint32_t mslot) {
        if constexpr (SH) {
            svr[0] = ds_read2<KQ_BSLOT(0) * kWsStride>(ws_lane + mslot);
            svr[1] = ds_read2<KQ_BSLOT(1) * kWsStride>(ws_lane + mslot);
            svr[2] = ds_read2<KQ_BSLOT(2) * kWsStride>(ws_lane + mslot);
            svr[3] = ds_read2<KQ_BSLOT(3) * kWsStride>(ws_lane + mslot);
        } else {
            svr[0] = ds_read4<KQ_BSLOT(0) * kWsStride>(ws_lane + mslot);
            svr[1] = ds_read4<KQ_BSLOT(1) * kWsStride>(ws_lane + mslot);
            svr[2] = ds_read4<KQ_BSLOT(2) * kWsStride>(ws_lane + mslot);
            svr[3] = ds_read4<KQ_BSLOT(3) * kWsStride>(ws_lane + mslot);
        }
        if constexpr (QM != QUANT_STATIC) asr = ds_read16<0>(as_lane + mslot);
        if constexpr (DBG) lgkm_wait<0>(svr[0], svr[1], svr[2], svr[3], asr);
    };
    // A register read from LDS is written when the data returns: until the covering lgkmcnt wait nothing may copy,
    // spill or reuse it. Every read here has a consumer behind a wait; the debug variant, which spills, waits at
    // once.
#define KQ_READ_A(mi, aslot)                                                       \
    do {                                                                           \
        A[mi][0] = ds_read16<(mi) * 16 * kBK>(a_lane0 + (aslot));                  \
        A[mi][1] = ds_read16<(mi) * 16 * kBK>(a_lane1 + (aslot));                  \
        if constexpr (DBG) lgkm_wait<0>(A[mi][0], A[mi][1]);                       \
    } while (0)
#define KQ_READ_B(ni, bslot)                                                       \
    do {                                                                           \
        B[ni][0] = ds_read16<(KQ_BSLOT(ni) * 2 + 0) * 1024>(b_lane + (bslot));     \
        B[ni][1] = ds_read16<(KQ_BSLOT(ni) * 2 + 1) * 1024>(b_lane + (bslot));     \
        if constexpr (DBG) lgkm_wait<0>(B[ni][0], B[ni][1]);                       \
    } while (0)
    // step kofs's operands
    read_meta(0);
    KQ_READ_A(0, 0);
    KQ_READ_A(1, 0);
    KQ_READ_A(2, 0);
    KQ_READ_B(0, 0);
    KQ_READ_B(1, 0);
    KQ_READ_B(2, 0);
    KQ_READ_B(3, 0);
    KQ_READ_A(3, 0);

    float sv[4], asel[4];  // weight and activation scales of the current step
    // Dynamic activations with F16 weight scales: the MFMAs of a group start from the bits of 1.5 * 2^23 instead of 0,
    // so the int32 accumulator holds 0x4B400000 + P', which read as f32 is exactly 12582912 + P' (|P'| < 2^22). One
    // FMA, (12582912 + P') * s + nb with nb = -12582912 * s, then gives round(s * P') -- the reference's t = s * P'
    // bit for bit: s comes from an F16 value (at most 11 significant bits), so nb is exact, and the FMA rounds the
    // exact s * P' once. acc += a_s * t is the second instruction (v_fmac with a DPP quad broadcast of a_s), two VALU
    // per element and group instead of three (conversion, product of the scales, FMA).
    constexpr bool kBias = SH && QM != QUANT_STATIC;
    constexpr float kBiasF = 12582912.0F;
    // The bias tuple comes out of inline assembly once, so the compiler keeps it in registers instead of
    // rematerializing the constant (a VALU write) in front of an MFMA that reads it: the hazard recognizer does not
    // see the MFMA inside the assembly and would not separate the two by the 2 wait states such a read needs.
    v4i biasv = {0, 0, 0, 0};
    if constexpr (kBias) {
        int b0 = 0, b1 = 0, b2 = 0, b3 = 0;  // (the host pass compiles the assembly out)
        KQ_ASM("v_mov_b32 %0, 0x4b400000\n\tv_mov_b32 %1, 0x4b400000\n\tv_mov_b32 %2, 0x4b400000\n\tv_mov_b32 %3, 0x4b400000"
               : "=v"(b0), "=v"(b1), "=v"(b2), "=v"(b3));
        biasv = v4i{b0, b1, b2, b3};
    }
    (void)biasv;
    float nbv[4];
    // Block b: two int8 MFMAs give the exact partials P' of the step's group. The epilogue of block b, issued after
    // the MFMAs of block b + 1, forms k = a_s * s in the accumulator's lane layout (lane = column nn + 16 L,
    // register r = row 4 L + r): the lane quad 4 (lane / 4) .. + 3 holds a_s of rows 16 mi + 4 L + 0..3 (one per
    // lane), so v_mul_f32 with a DPP quad broadcast of lane r gives k[r] in one VALU instruction (an f32 4x4x1 MFMA
    // for the same products costs more issue time, measured); then acc += k * P' (cvt, fmac).
    auto mfmas = [&](int blk, v4i& c) {
        const int mi = blk >> 2, ni = blk & 3;
        // reads return in order: after B0 come B1, B2, B3 and A3 (8 reads)
        if (blk == 0) {
            lgkm_wait<8>(svr[0], svr[1], svr[2], svr[3], asr, A[0][0], A[0][1], A[1][0], A[1][1], A[2][0], A[2][1], B[0][0], B[0][1]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sv[i] = SH ? __half2float(__ushort_as_half(static_cast<unsigned short>(svr[i]))) : __uint_as_float(svr[i]);
                asel[i] = __int_as_float(asr[i]);
                if constexpr (kBias) nbv[i] = -kBiasF * sv[i];
            }
        }
        if (blk == 1) lgkm_wait<6>(B[1][0], B[1][1]);
        if (blk == 2) lgkm_wait<4>(B[2][0], B[2][1]);
        if (blk == 3) lgkm_wait<2>(B[3][0], B[3][1]);
        if (blk == 4) lgkm_wait<0>(A[3][0], A[3][1]);
#if defined(__HIP_DEVICE_COMPILE__)
        if constexpr (!DBG) {
            // issue order pinned (see the epilogue)
            if constexpr (kBias)
                KQ_ASM("v_mfma_i32_16x16x64_i8 %0, %1, %2, %3" : "=&v"(c) : "v"(A[mi][0]), "v"(B[ni][0]), "v"(biasv));
            else
                KQ_ASM("v_mfma_i32_16x16x64_i8 %0, %1, %2, 0" : "=&v"(c) : "v"(A[mi][0]), "v"(B[ni][0]));
            KQ_ASM("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+v"(c) : "v"(A[mi][1]), "v"(B[ni][1]));
            return;
        }
#endif
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mi][0], B[ni][0], zero, 0, 0, 0);
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mi][1], B[ni][1], c, 0, 0, 0);
    };
    auto epilogue = [&](const v4i& c, int blk, int kt) {
        const int mi = blk >> 2, ni = blk & 3;
#if defined(__HIP_DEVICE_COMPILE__)
        if constexpr (!DBG) {
            // Inline assembly keeps this block's products, conversions and FMAs after the MFMAs of the next block (the
            // compiler would pull them up behind their own MFMAs and stall on the results); by then at least ten
            // instructions separate every MFMA result from its first VALU read, beyond the dependency window.
            // (asel is last written at the step's first block, long before these DPP reads.)
            float kk[4], t[4];
            if constexpr (kBias) {
#pragma unroll
                for (int r = 0; r < 4; ++r) KQ_ASM("v_fma_f32 %0, %1, %2, %3" : "=v"(t[r]) : "v"(c[r]), "v"(sv[ni]), "v"(nbv[ni]));
                KQ_ASM("v_fmac_f32_dpp %0, %1, %2 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf" : "+v"(acc[mi][ni][0]) : "v"(asel[mi]), "v"(t[0]));
                KQ_ASM("v_fmac_f32_dpp %0, %1, %2 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf" : "+v"(acc[mi][ni][1]) : "v"(asel[mi]), "v"(t[1]));
                KQ_ASM("v_fmac_f32_dpp %0, %1, %2 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf" : "+v"(acc[mi][ni][2]) : "v"(asel[mi]), "v"(t[2]));
                KQ_ASM("v_fmac_f32_dpp %0, %1, %2 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf" : "+v"(acc[mi][ni][3]) : "v"(asel[mi]), "v"(t[3]));
                return;
            }
            if constexpr (QM == QUANT_STATIC) {
#pragma unroll
                for (int r = 0; r < 4; ++r) kk[r] = sv[ni];
            } else {
                KQ_ASM("v_mul_f32_dpp %0, %1, %2 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf" : "=v"(kk[0]) : "v"(asel[mi]), "v"(sv[ni]));
                KQ_ASM("v_mul_f32_dpp %0, %1, %2 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf" : "=v"(kk[1]) : "v"(asel[mi]), "v"(sv[ni]));
                KQ_ASM("v_mul_f32_dpp %0, %1, %2 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf" : "=v"(kk[2]) : "v"(asel[mi]), "v"(sv[ni]));
                KQ_ASM("v_mul_f32_dpp %0, %1, %2 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf" : "=v"(kk[3]) : "v"(asel[mi]), "v"(sv[ni]));
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) KQ_ASM("v_cvt_f32_i32 %0, %1" : "=v"(t[r]) : "v"(c[r]));
#pragma unroll
            for (int r = 0; r < 4; ++r) KQ_ASM("v_fmac_f32 %0, %1, %2" : "+v"(acc[mi][ni][r]) : "v"(kk[r]), "v"(t[r]));
            return;
        }
#endif
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int P = c[r];
            if (DBG && a.dump) {
                const int row = m0 + wm * 64 + mi * 16 + 4 * L + r, col = col_nt[ni] * kTileRows + nn;
                if (row < a.M && col_nt[ni] < a.n_tiles && col < a.N)
                    a.dump[(static_cast<std::int64_t>(row) * a.N + col) * a.groups + kt] = P;
            }
            float kk = sv[ni];
            if constexpr (QM != QUANT_STATIC) {
                // a_s of row 16 mi + 4 L + r: quad lane r's value (quad_perm [r, r, r, r])
                const int ctrl = 0x55 * r;
                const int bits = __float_as_int(asel[mi]);
                const int rs = ctrl == 0 ? __builtin_amdgcn_mov_dpp(bits, 0x00, 0xF, 0xF, false)
                               : ctrl == 0x55 ? __builtin_amdgcn_mov_dpp(bits, 0x55, 0xF, 0xF, false)
                               : ctrl == 0xAA ? __builtin_amdgcn_mov_dpp(bits, 0xAA, 0xF, 0xF, false)
                                              : __builtin_amdgcn_mov_dpp(bits, 0xFF, 0xF, 0xF, false);
                if constexpr (kBias) {  // the biased form's arithmetic: t = s * P' rounded once, acc += a_s * t fused
                    const float t = sv[ni] * static_cast<float>(P);
                    acc[mi][ni][r] = __builtin_fmaf(__int_as_float(rs), t, acc[mi][ni][r]);
                    continue;
                }
                kk = __int_as_float(rs) * sv[ni];
            }
            acc[mi][ni][r] = __builtin_fmaf(kk, static_cast<float>(P), acc[mi][ni][r]);
        }
    };
    auto sched_blocks = [&]() {
        if constexpr (!DBG) {
            // one block: 2 MFMAs, then the VALU of the previous block's epilogue (12; 8 with static activations or
            // the biased accumulators)
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, (QM == QUANT_STATIC || kBias) ? 8 : 12, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    v4i cp;  // MFMA results of the block whose epilogue is pending
    // First half of step kt (slot s1 = step kt + 1): blocks 0-7, step kt + 1's tiles unpacked into B slot
    // (kt + 1) % 2, then the step's barrier.
    auto phase1 = [&](int kt, int s1) {
        v4i cn;
        Raw raw;
        mfmas(0, cp);
#pragma unroll
        for (int blk = 1; blk < 8; ++blk) {
            mfmas(blk, cn);
            if (blk == 4) raw = unpack_read(s1, s1);
            if (blk == 6) unpack_write(raw, (kt - kofs + 1) & 1);
            // block 0's partials: only block 1's MFMAs lie between them and their first VALU read, fewer than the
            // 8 wait states an int8 MFMA result needs (the hazard recognizer does not see into inline assembly)
            if (blk == 1 && !DBG) KQ_ASM("s_nop 7");
            epilogue(cp, blk - 1, kt);
            cp = cn;
        }
        sched_blocks();
        // all LDS traffic of the loop is explicit: the wait covers it, so a bare barrier (no fence) suffices
        __builtin_amdgcn_s_waitcnt(kStepWait);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    // Second half of step kt (slots s0 = step kt, s1 = step kt + 1): blocks 8-15; copies of step kt + 3 (activation
    // codes, metadata) and kt + 4 (packed tiles, zero points); step kt + 1's operand registers read after their
    // last use here (not after the last step: a read nobody waits for would land in a register by then reused).
    auto phase2 = [&](int kt, int s0, int s1, bool next) {
        const int k3 = clamp_k(kt + 3), k4 = clamp_k(kt + 4);
        const std::uint32_t aslot1 = s1 * S::A_BYTES, mslot1 = s1 * S::META_BYTES;
        const std::uint32_t bslot1 = ((kt - kofs + 1) & 1) * kBBytes;
        v4i cn;
        if (next) {
            read_meta(mslot1);
            KQ_READ_A(0, aslot1);
            KQ_READ_A(1, aslot1);
        }
#pragma unroll
        for (int blk = 8; blk <= 16; ++blk) {
            if (blk < 16) mfmas(blk, cn);
            if (blk <= 11) issue_a(k3, s0, blk - 8);
            if (blk == 12) {
                issue_raw(k4, s1);
                if (next) KQ_READ_A(2, aslot1);
            }
            if (blk == 13) {
                issue_meta(k3, s0, k4, s1);
                if (next) KQ_READ_B(0, bslot1);
            }
            if (next && blk == 14) KQ_READ_B(1, bslot1);
            if (next && blk == 15) KQ_READ_B(2, bslot1);
            if (next && blk == 16) {
                KQ_READ_B(3, bslot1);
                KQ_READ_A(3, aslot1);
            }
            epilogue(cp, blk - 1, kt);
            if (blk < 16) cp = cn;
        }
        sched_blocks();
    };

    // one iteration: second half of step kt, first half of step kt + 1 (its barrier ends the iteration), so every
    // register read from LDS is complete before the loop's back edge
    phase1(kofs, 1);
    int s0 = 0, s1 = 1;  // ring slots (mod 3) of steps kt and kt + 1
    for (int kt = kofs; kt < kend - 1; ++kt) {
        const int s2 = s1 == 2 ? 0 : s1 + 1;
        phase2(kt, s0, s1, true);
        phase1(kt + 1, s2);
        s0 = s1;
        s1 = s2;
    }
    phase2(kend - 1, s0, s1, false);
#undef KQ_BSLOT
#undef KQ_READ_A
#undef KQ_READ_B
    // no copy or read may still be in flight when the workgroup's LDS is handed to the next workgroup
    __builtin_amdgcn_s_waitcnt(0);

    if (a.ksplit > 1) {
        // K-split: every range stores its fp32 partial tile, as [16 groups (mi, ni)][thread] of float4 so each store
        // of a wave is 1 KiB contiguous; gemm_i4_reduce_kernel adds the ranges in range order
        float* const dst = a.partial + (static_cast<std::int64_t>(ks) * tiles + tile) * S::THREADS * 64 + tid * 4;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                __builtin_nontemporal_store(v4f{acc[mi][ni][0], acc[mi][ni][1], acc[mi][ni][2], acc[mi][ni][3]},
                                            reinterpret_cast<v4f*>(dst + (mi * 4 + ni) * S::THREADS * 4));
        return;
    }
    store_tile<WM, GELU, QM>(a, acc, m0, col_nt, wm, nn, L);
}

// Sum of the K ranges of one output tile (range order, so the result does not depend on which range finished
// first), then the same epilogue as the unsplit GEMM. Four workgroups per output tile, one per 16-row strip mi of
// every wave's 64 x 64 block; threads as in the GEMM.
template <int WM, bool GELU, int QM>
__global__ __launch_bounds__(GemmShape<WM>::THREADS) void gemm_i4_reduce_kernel(GemmArgs a) {
    using S = GemmShape<WM>;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int nn = lane & 15, L = lane >> 4;
    const int tiles = a.m_blocks * a.n_blocks, tile = blockIdx.x >> 2, strip = blockIdx.x & 3;
    const int mb = tile % a.m_blocks, nb = tile / a.m_blocks;
    int col_nt[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) col_nt[ni] = slot_tile<GELU>(a, nb, wave_slot<GELU>(wn, ni));
    float acc[4][4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mi][ni][r] = 0.F;
    for (int q = 0; q < a.ksplit; ++q) {
        const float* src = a.partial + (static_cast<std::int64_t>(q) * tiles + tile) * S::THREADS * 64 + tid * 4;
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(src + (strip * 4 + ni) * S::THREADS * 4));
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                if (mi != strip) continue;
                acc[mi][ni][0] = acc[mi][ni][0] + v[0];
                acc[mi][ni][1] = acc[mi][ni][1] + v[1];
                acc[mi][ni][2] = acc[mi][ni][2] + v[2];
                acc[mi][ni][3] = acc[mi][ni][3] + v[3];
            }
        }
    }
    store_tile<WM, GELU, QM>(a, acc, mb * S::BM, col_nt, wm, nn, L, strip);
}

__global__ __launch_bounds__(256) void unpermute_rows_kernel(const std::int8_t* q, int M, int K, std::int8_t* codes) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= static_cast<std::int64_t>(M) * K) return;
    const std::int64_t m = id / K, k = id % K;
    codes[id] = q[m * K + act_position(k)];
}

__global__ __launch_bounds__(256) void transpose_stats_kernel(const float* s_t, const std::int32_t* q_t, int M, int M_p,
                                                              int groups, float* s, std::int32_t* q, std::int32_t* z) {
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= M * groups) return;
    const int m = id / groups, b = id % groups;
    if (s) s[id] = s_t[b * M_p + scale_slot(m)];
    if (q) q[id] = q_t[b * M_p + scale_slot(m)];
    if (z) z[id] = 0;
}

}  // namespace

// Launch plan: 256-row tiles (WM = 4), the K range split in 2, 4 or 8 when that fills the chip (at least 256
// workgroups) and every range keeps >= 16 groups; otherwise 128-row tiles (WM = 2), split the same way. A split adds
// one small reduction launch and the partial tiles' traffic, so short K ranges do not pay for it.
GemmPlan gemm_i4_plan(const Weight& w, std::int64_t M, bool gelu) {
    const int kt = static_cast<int>(w.geo.k_tiles);
    GemmPlan p;
    p.n_blocks = gelu ? static_cast<int>((w.geo.n_tiles / 2 + 3) / 4) : static_cast<int>((w.geo.n_tiles + 7) / 8);
    auto blocks_m = [&](int wm) { return static_cast<int>((M + 64 * wm - 1) / (64 * wm)); };
    auto best_split = [&](int tiles, bool need_full) {
        int best = 0;
        for (int sp = 1; sp <= 8; sp *= 2) {
            if (kt % sp || (sp > 1 && kt / sp < 16)) break;
            best = sp;
            if (tiles * sp >= 256) return sp;
        }
        return need_full ? 0 : best;
    };
    p.wm = 4;
    p.m_blocks = blocks_m(4);
    p.ksplit = best_split(p.m_blocks * p.n_blocks, true);
    if (p.ksplit == 0) {
        p.wm = 2;
        p.m_blocks = blocks_m(2);
        p.ksplit = best_split(p.m_blocks * p.n_blocks, false);
    }
    if (p.ksplit < 1) p.ksplit = 1;
    return p;
}

bool gemm_i4_fits(const LinearCall& c) {
    const Weight& w = *c.w;
    if (!w.tiled || w.geo.bits != 4 || w.geo.group != 128 || c.M <= 16) return false;
    if (c.path != PATH_BLOCKWISE && c.path != PATH_SYMMETRIC) return false;
    if (w.zero_mode == ZERO_FLOAT) return false;
    if (w.geo.cols % 512 || w.geo.cols_p != w.geo.cols) return false;
    if (c.gelu_gate && ((w.geo.rows / 2) % kTileRows || w.geo.n_tiles % 2)) return false;
    const std::int64_t M_p = round_up(c.M, kQuantRows);
    // the row quantizer addresses x with 32-bit byte offsets (buffer resource of M * K * element bytes)
    if (c.M * w.geo.cols * (c.x_type == ACT_F32 ? 4 : 2) >= (std::int64_t{1} << 32)) return false;
    if (M_p * w.geo.cols >= (std::int64_t{1} << 31) || w.geo.k_tiles * kTileBytes >= (std::int64_t{1} << 31) ||
        w.geo.meta_count() * 4 >= (std::int64_t{1} << 31) || M_p * w.geo.groups_p * 4 >= (std::int64_t{1} << 31))
        return false;
    return true;
}

std::int64_t gemm_i4_rows(std::int64_t M) { return round_up(M, kQuantRows); }

hipError_t launch_gemm_i4(const LinearCall& c, const ActBuffers& act, hipStream_t stream) {
    const Weight& w = *c.w;
    const int M = static_cast<int>(c.M), K = static_cast<int>(w.geo.cols);
    const int M_p = static_cast<int>(gemm_i4_rows(c.M));
    const bool stat = c.path == PATH_SYMMETRIC;
    QRowArgs q{};
    q.x = c.x;
    q.x_f32 = c.x_type == ACT_F32;
    q.M = M;
    q.M_p = M_p;
    q.K = K;
    q.input_scale = c.input_scale;
    q.q = act.q;
    q.scale_t = act.scale;
    q.sum_t = nullptr;
    q.ninv = c.norm_inv;
    q.nw = c.norm_inv ? c.norm_w1 : nullptr;
    const GemmPlan plan = gemm_i4_plan(w, c.M, c.gelu_gate);
    launch_quantize_rows(q, stat, q.x_f32 != 0, stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;

    GemmArgs a{};
    a.q = act.q;
    a.scale_t = act.scale;
    a.tiles = w.tiles;
    a.scales = w.scales;
    a.zero_points = w.zero_mode == ZERO_POINT ? w.zero_points : nullptr;
    a.y = c.y;
    a.dump = c.dump;
    a.M = M;
    a.M_p = M_p;
    a.N = static_cast<int>(w.geo.rows);
    a.K = K;
    a.k_tiles = static_cast<int>(w.geo.k_tiles);
    a.n_tiles = static_cast<int>(w.geo.n_tiles);
    a.groups_p = static_cast<int>(w.geo.groups_p);
    a.groups = static_cast<int>(w.geo.cols / w.geo.group);
    a.scale_half = w.scale_type == META_F16;
    a.input_scale = c.input_scale;
    a.output_scale = c.output_scale;
    const int wm = plan.wm;
    a.m_blocks = plan.m_blocks;
    a.n_blocks = plan.n_blocks;
    a.ksplit = plan.ksplit;
    a.partial = act.partial;
    if (plan.ksplit > 1 && !act.partial) return hipErrorInvalidValue;
    const bool zp = w.zero_mode == ZERO_POINT;
    const bool dbg = c.dump != nullptr;
    const bool sh = w.scale_type == META_F16;
    const dim3 grid(static_cast<unsigned>(a.m_blocks * a.n_blocks * a.ksplit));
#define KQ_G(WM, GE, QM, Z, H, D) \
    hipLaunchKernelGGL((gemm_i4_kernel<WM, GE, QM, Z, H, D>), grid, dim3(GemmShape<WM>::THREADS), GemmShape<WM>::LDS, stream, a)
#define KQ_GH(WM, GE, QM, Z, D) \
    if (sh) KQ_G(WM, GE, QM, Z, true, D); \
    else KQ_G(WM, GE, QM, Z, false, D)
#define KQ_GW(GE, QM, Z, D) \
    if (wm == 4) { KQ_GH(4, GE, QM, Z, D); } \
    else { KQ_GH(2, GE, QM, Z, D); }
    if (stat) {
        if (c.gelu_gate) { KQ_GW(true, dev::QUANT_STATIC, false, false) }
        else if (dbg) { KQ_GW(false, dev::QUANT_STATIC, false, true) }
        else { KQ_GW(false, dev::QUANT_STATIC, false, false) }
    } else if (zp) {
        if (c.gelu_gate) { KQ_GW(true, dev::QUANT_DYN_SYM, true, false) }
        else if (dbg) { KQ_GW(false, dev::QUANT_DYN_SYM, true, true) }
        else { KQ_GW(false, dev::QUANT_DYN_SYM, true, false) }
    } else {
        if (c.gelu_gate) { KQ_GW(true, dev::QUANT_DYN_SYM, false, false) }
        else if (dbg) { KQ_GW(false, dev::QUANT_DYN_SYM, false, true) }
        else { KQ_GW(false, dev::QUANT_DYN_SYM, false, false) }
    }
#undef KQ_GW
#undef KQ_GH
#undef KQ_G
    e = hipGetLastError();
    if (e != hipSuccess || plan.ksplit == 1) return e;
    const dim3 rgrid(static_cast<unsigned>(a.m_blocks * a.n_blocks * 4));
#define KQ_R(WM, GE, QM) hipLaunchKernelGGL((gemm_i4_reduce_kernel<WM, GE, QM>), rgrid, dim3(GemmShape<WM>::THREADS), 0, stream, a)
#define KQ_RW(GE, QM) \
    if (wm == 4) KQ_R(4, GE, QM); \
    else KQ_R(2, GE, QM)
    if (stat) {
        if (c.gelu_gate) { KQ_RW(true, dev::QUANT_STATIC); }
        else { KQ_RW(false, dev::QUANT_STATIC); }
    } else {
        if (c.gelu_gate) { KQ_RW(true, dev::QUANT_DYN_SYM); }
        else { KQ_RW(false, dev::QUANT_DYN_SYM); }
    }
#undef KQ_RW
#undef KQ_R
    return hipGetLastError();
}

// Quantizer outputs of the prefill path in the debug form (natural-order codes [M][K], stats [M][K/g]).
hipError_t launch_gemm_i4_quantize_dump(const LinearCall& c, const ActBuffers& act, std::int8_t* codes, float* scales,
                                        std::int32_t* sums, std::int32_t* zero_points, hipStream_t stream) {
    const Weight& w = *c.w;
    const int M = static_cast<int>(c.M), K = static_cast<int>(w.geo.cols);
    const int M_p = static_cast<int>(gemm_i4_rows(c.M));
    QRowArgs q{};
    q.x = c.x;
    q.x_f32 = c.x_type == ACT_F32;
    q.M = M;
    q.M_p = M_p;
    q.K = K;
    q.input_scale = c.input_scale;
    q.q = act.q;
    q.scale_t = act.scale;
    q.sum_t = act.sum;
    launch_quantize_rows(q, c.path == PATH_SYMMETRIC, q.x_f32 != 0, stream);
    const std::int64_t total = static_cast<std::int64_t>(M) * K;
    if (codes) hipLaunchKernelGGL(unpermute_rows_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, act.q, M, K, codes);
    const int groups = K / 128;
    hipLaunchKernelGGL(transpose_stats_kernel, dim3(static_cast<unsigned>((M * groups + 255) / 256)), dim3(256), 0, stream,
                       act.scale, act.sum, M, M_p, groups, scales, sums, zero_points);
    return hipGetLastError();
}

}  // namespace kq
