// Prefill projection (M > 16) for 4-bit weights with small groups, g = 32 or 64 (the fused QKV of a decoder layer is
// g = 32): Kidi's BlockwiseLinear / SymmetricPackedLinear closed forms (runtime/ynn/operators.cpp:1118-1169,
// :1250-1308) over int8 activation codes from quantize_rows_g_kernel ([M_p][K] in the tiles' permuted order, block
// scales [K/g][M_p]).
//
// Workgroup tile 128 rows x 128 output columns (8 weight row tiles), 8 waves of 32 x 64 (8 blocks of 16 x 16), one
// 128-column k step per iteration = 128/g groups. LDS holds two stages; each step the next step's operands travel
// global -> registers (issued before the step's MFMAs) -> LDS (after them): activation codes XOR-swizzled by row so
// the A-operand reads spread over the banks, packed int4 tiles unpacked to int8 with the zero point of each byte's
// group folded in (byte = u - zp), weight scales as f32 [group][wave column][row][tile], activation scales
// [group][128 rows]. Per 16 x 16 block and group: one int8 MFMA gives the exact partial P' = sum q (u - zp) of the
// group (v_mfma_i32_16x16x32_i8 on the 8 bytes of a lane that belong to a 32-column group, v_mfma_i32_16x16x64_i8
// for g = 64), and the epilogue is k = a_s * s (v_mul), acc += k * P' (cvt, fmac). The epilogue runs once per
// group, so small groups make this kernel VALU-bound: three VALU per output element and group against one int8
// MFMA over 32 or 64 columns.
// Two workgroups fit a CU (72 KB of LDS at g = 32, at most 128 VGPRs), so a 2048 x 2560 projection (320 tiles) runs
// in one wave of workgroups, and every SIMD holds at least two waves (one wave issues a VALU at most every other
// slot).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kq_device.hpp"
#include "kq_internal.hpp"

namespace kq {
namespace {

using namespace dev;

typedef float v4f __attribute__((ext_vector_type(4)));

// (the host pass sees the kernel bodies too; the assembly is device-only)
#if defined(__HIP_DEVICE_COMPILE__)
#define KQ_GASM(...) asm volatile(__VA_ARGS__)
#else
#define KQ_GASM(...) (void)0
#endif

constexpr int kBM = 128, kBK = 128, kSlots = 8;  // rows, columns per step, row tiles per workgroup
constexpr int kWaves = 8;  // two per SIMD in every workgroup: a lone workgroup on a CU still issues VALU at the
                           // two-wave rate (one wave issues a VALU at most every other slot)

template <int G>
struct GShape {
    static constexpr int GPS = kBK / G;                  // groups per step
    static constexpr int A_BYTES = kBM * kBK;            // codes [row][128], 16-byte chunks swizzled
    static constexpr int B_BYTES = kSlots * 2048;        // unpacked int8 [slot][64-column half][lane][16 B]
    static constexpr int WS_BYTES = GPS * 2 * 16 * 4 * 4;  // f32 [group][wave column][row nn][tile ni]
    static constexpr int AS_BYTES = GPS * kBM * 4;       // f32 [group][row]
    static constexpr int B_OFF = A_BYTES, WS_OFF = B_OFF + B_BYTES, AS_OFF = WS_OFF + WS_BYTES;
    static constexpr int STAGE = AS_OFF + AS_BYTES;
    static constexpr int LDS = 2 * STAGE;
    static_assert(LDS <= 80 * 1024, "two workgroups per CU");
};

// Waves of a workgroup: 2 columns of 64 output columns x WAVES/2 rows of WR output rows (MI blocks of 16 rows).
template <int WAVES>
struct GWaves {
    static constexpr int THREADS = 64 * WAVES, WR = kBM / (WAVES / 2), MI = WR / 16;
    static constexpr int A_PER = kBM * kBK / 16 / THREADS;  // 16-byte activation chunks per thread
    static constexpr int B_PER = kSlots * 64 / THREADS;     // 16-byte packed-tile lane slots per thread
};

struct GArgs {
    const std::int8_t* q;      // [M_p][K] permuted codes
    const float* a_scale;      // [groups_p][M_p] (rows contiguous: a step's 128 rows are one coalesced read)
    const std::uint8_t* tiles;
    const void* scales;        // [n_tiles][groups_p][16] F16|F32
    const std::uint8_t* zero_points;  // [n_tiles][groups_p][8] nibble pairs, or null (symmetric: 8)
    float* y;
    std::int32_t* dump;        // optional int32 partials [M][N][groups]
    int M, M_p, N, K, k_tiles, n_tiles, groups_p, groups;
    float input_scale, output_scale;
    int m_blocks, n_blocks;
};

template <int G, int QM, bool ZP, bool SH, bool DBG, int WAVES>
__global__ __launch_bounds__(64 * WAVES, WAVES / 2) void gemm_i4g_kernel(GArgs a) {
    using S = GShape<G>;
    using WV = GWaves<WAVES>;
    constexpr int GPS = S::GPS, T = WV::THREADS, MI = WV::MI;
    constexpr int META_PER_THREAD = (GPS * kBM + T - 1) / T;  // weight scales (and activation scales) per thread
    extern __shared__ __attribute__((aligned(16))) std::uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % (WAVES / 2), wn = wave / (WAVES / 2);
    const int nn = lane & 15, L = lane >> 4;

    // workgroup -> tile; each XCD (every 8th workgroup) takes a contiguous range of tiles, column-block major, so its
    // L2 holds few weight column blocks
    const int total = a.m_blocks * a.n_blocks;
    int bid = blockIdx.x;
    if (total % 8 == 0) bid = (bid % 8) * (total / 8) + bid / 8;
    const int mb = bid % a.m_blocks, nb = bid / a.m_blocks;
    const int m0 = mb * kBM;

    // ---- per-thread copy assignments (fixed for the whole K loop) ----
    // activation codes: chunks c = tid + T i of 16 bytes, row c / 8, chunk c % 8
    const std::int8_t* a_src[WV::A_PER];
    int a_dst[WV::A_PER];
#pragma unroll
    for (int i = 0; i < WV::A_PER; ++i) {
        const int c = tid + T * i, r = c >> 3, ch = c & 7;
        a_src[i] = a.q + static_cast<std::int64_t>(m0 + r) * a.K + ch * 16;
        a_dst[i] = r * kBK + ((ch ^ (r & 7)) << 4);
    }
    // packed tiles: lane slots c = tid + T i of the 8 tiles: tile slot c / 64, lane slot s = c % 64 (row s % 16)
    const std::uint8_t* b_src[WV::B_PER];
    int b_nt[WV::B_PER], b_dst[WV::B_PER], b_row[WV::B_PER];
#pragma unroll
    for (int i = 0; i < WV::B_PER; ++i) {
        const int c = tid + T * i, t = c >> 6, s = c & 63;
        const int nt = nb * kSlots + t;
        b_nt[i] = nt < a.n_tiles ? nt : -1;
        b_src[i] = a.tiles + static_cast<std::int64_t>(nt < a.n_tiles ? nt : 0) * a.k_tiles * kTileBytes + s * 16;
        b_dst[i] = S::B_OFF + t * 2048 + s * 16;
        b_row[i] = s & 15;
    }
    // metadata: values v = tid + T i < 128 GPS: group v / 128, then (weight scales) tile slot (v / 16) % 8 and row
    // v % 16, or (activation scales) row v % 128
    int m_g[META_PER_THREAD], m_t[META_PER_THREAD], m_r[META_PER_THREAD];
    bool m_live[META_PER_THREAD];
#pragma unroll
    for (int i = 0; i < META_PER_THREAD; ++i) {
        const int v = tid + T * i;
        m_live[i] = v < GPS * kBM;
        m_g[i] = m_live[i] ? v >> 7 : 0;
        m_t[i] = (v >> 4) & 7;
        m_r[i] = v & 127;
    }

    // the next step's operands, held in registers while the current step computes
    v4u pa[WV::A_PER], pb[WV::B_PER];
    std::uint32_t pz[WV::B_PER][GPS];
    float pws[META_PER_THREAD], pas[META_PER_THREAD];
    auto load = [&](int k) {
#pragma unroll
        for (int i = 0; i < WV::A_PER; ++i) pa[i] = *reinterpret_cast<const v4u*>(a_src[i] + k * kBK);
#pragma unroll
        for (int i = 0; i < WV::B_PER; ++i) {
            pb[i] = b_nt[i] >= 0 ? __builtin_nontemporal_load(reinterpret_cast<const v4u*>(b_src[i] + static_cast<std::int64_t>(k) * kTileBytes))
                                 : v4u{0u, 0u, 0u, 0u};
#pragma unroll
            for (int h = 0; h < GPS; ++h) {
                pz[i][h] = 8;
                if (ZP && b_nt[i] >= 0)
                    pz[i][h] = a.zero_points[(static_cast<std::int64_t>(b_nt[i]) * a.groups_p + k * GPS + h) * 8 + (b_row[i] >> 1)];
            }
        }
#pragma unroll
        for (int i = 0; i < META_PER_THREAD; ++i) {
            const int nt = nb * kSlots + m_t[i];
            float s = 0.F;
            if (m_live[i] && nt < a.n_tiles) {
                const std::int64_t mi = (static_cast<std::int64_t>(nt) * a.groups_p + k * GPS + m_g[i]) * kTileRows + (m_r[i] & 15);
                s = SH ? __half2float(static_cast<const __half*>(a.scales)[mi]) : static_cast<const float*>(a.scales)[mi];
            }
            pws[i] = s;
            pas[i] = (QM == QUANT_STATIC || !m_live[i]) ? 0.F : a.a_scale[static_cast<std::int64_t>(k * GPS + m_g[i]) * a.M_p + m0 + m_r[i]];
        }
    };
    auto store = [&](int stage) {
        std::uint8_t* st = lds + stage * S::STAGE;
#pragma unroll
        for (int i = 0; i < WV::A_PER; ++i) *reinterpret_cast<v4u*>(st + a_dst[i]) = pa[i];
#pragma unroll
        for (int i = 0; i < WV::B_PER; ++i) {
            // 64-column half j: dwords 2j, 2j + 1 hold its 16 codes (low nibbles, then high nibbles); bytes 0-7 of
            // the unpacked half are its first 32 columns, bytes 8-15 the second
            const std::uint32_t w[4] = {pb[i].x, pb[i].y, pb[i].z, pb[i].w};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                std::uint32_t z0, z1;  // zero point (in every byte) of bytes 0-7 and of bytes 8-15
                if constexpr (G == 32) {
                    z0 = (pz[i][2 * j] >> (4 * (b_row[i] & 1))) & 15u;
                    z1 = (pz[i][2 * j + 1] >> (4 * (b_row[i] & 1))) & 15u;
                } else {
                    z0 = z1 = (pz[i][j] >> (4 * (b_row[i] & 1))) & 15u;
                }
                if (!ZP) z0 = z1 = 8u;
                const std::uint32_t zz0 = z0 * 0x01010101u, zz1 = z1 * 0x01010101u;
                const std::uint32_t d0 = w[2 * j], d1 = w[2 * j + 1];
                uint4 o;
                o.x = (((d0 & 0x0F0F0F0Fu) | 0x80808080u) - zz0) ^ 0x80808080u;
                o.y = ((((d0 >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zz0) ^ 0x80808080u;
                o.z = (((d1 & 0x0F0F0F0Fu) | 0x80808080u) - zz1) ^ 0x80808080u;
                o.w = ((((d1 >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zz1) ^ 0x80808080u;
                *reinterpret_cast<uint4*>(st + b_dst[i] + j * 1024) = o;
            }
        }
        float* ws = reinterpret_cast<float*>(st + S::WS_OFF);
        float* as = reinterpret_cast<float*>(st + S::AS_OFF);
#pragma unroll
        for (int i = 0; i < META_PER_THREAD; ++i) {
            if (!m_live[i]) continue;
            ws[((m_g[i] * 2 + (m_t[i] >> 2)) * 16 + (m_r[i] & 15)) * 4 + (m_t[i] & 3)] = pws[i];
            as[m_g[i] * kBM + m_r[i]] = pas[i];
        }
    };

    float acc[MI][4][4];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mi][ni][r] = 0.F;
    const v4f zerof = {0.F, 0.F, 0.F, 0.F};
    const v4i zero = {0, 0, 0, 0};
    // Dynamic activations with F16 weight scales: each group's MFMA starts from the bits of 1.5 * 2^23, so the
    // accumulator read as f32 is exactly 12582912 + P' (|P'| < 2^22), and fma(that, s, -12582912 * s) is round(s * P')
    // (-12582912 * s is exact for an s of at most 11 significant bits): the conversion and the weight scale in one
    // instruction, acc += a_s * t in a second. The bias registers come out of inline assembly once, so the compiler
    // keeps them instead of rematerializing the constant (a VALU write) just before an MFMA that reads it.
    constexpr bool kBias = SH && QM != QUANT_STATIC;
    constexpr float kBiasF = 12582912.0F;
    v4i biasv = zero;
    if constexpr (kBias) {
        int b0 = 0, b1 = 0, b2 = 0, b3 = 0;  // (the host pass compiles the assembly out)
        KQ_GASM("v_mov_b32 %0, 0x4b400000\n\tv_mov_b32 %1, 0x4b400000\n\tv_mov_b32 %2, 0x4b400000\n\tv_mov_b32 %3, 0x4b400000"
                : "=v"(b0), "=v"(b1), "=v"(b2), "=v"(b3));
        biasv = v4i{b0, b1, b2, b3};
    }
    (void)biasv;

    load(0);
    store(0);
    __syncthreads();

    for (int k = 0; k < a.k_tiles; ++k) {
        const bool more = k + 1 < a.k_tiles;
        if (more) load(k + 1);
        const std::uint8_t* st = lds + (k & 1) * S::STAGE;
        const float* ws = reinterpret_cast<const float*>(st + S::WS_OFF);
        const float* as = reinterpret_cast<const float*>(st + S::AS_OFF);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            v4i A[MI], B[4];
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
                const int row = wm * WV::WR + mi * 16 + nn;
                A[mi] = *reinterpret_cast<const v4i*>(st + row * kBK + (((4 * j + L) ^ (row & 7)) << 4));
            }
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                B[ni] = *reinterpret_cast<const v4i*>(st + S::B_OFF + (4 * wn + ni) * 2048 + j * 1024 + lane * 16);
            constexpr int HALVES = G == 32 ? 2 : 1;  // groups in this 64-column half
#pragma unroll
            for (int h = 0; h < HALVES; ++h) {
                const int gi = G == 32 ? 2 * j + h : j;  // group of the step
                const v4f sv4 = *reinterpret_cast<const v4f*>(ws + ((gi * 2 + wn) * 16 + nn) * 4);
                v4f nb4 = zerof;
                if constexpr (kBias) nb4 = sv4 * -kBiasF;
                (void)nb4;
                v4f as4[MI];  // activation scales of rows 16 mi + 4 L + r, r = 0..3 (the accumulator's rows)
#pragma unroll
                for (int mi = 0; mi < MI; ++mi) {
                    as4[mi] = zerof;
                    if constexpr (QM != QUANT_STATIC) as4[mi] = *reinterpret_cast<const v4f*>(as + gi * kBM + wm * WV::WR + 16 * mi + 4 * L);
                }
                // block blk = 4 mi + ni: one int8 MFMA gives the exact group partial; the epilogue forms a_s * s on
                // the VALU (four v_mul_f32: an f32 4x4x1 MFMA for the same products costs more issue time than the
                // multiplies), converts the partial and accumulates. MFMAs and epilogue are volatile assembly so
                // their issue order stays as written (the compiler would hoist every MFMA of the step above the first
                // epilogue and spill the results); the debug variant, which stores partials, uses the builtins.
                auto mfmas = [&](int blk, v4i& c) {
                    const int mi = blk >> 2, ni = blk & 3;
                    const long av = (static_cast<long>(static_cast<std::uint32_t>(A[mi][2 * h + 1])) << 32) |
                                    static_cast<std::uint32_t>(A[mi][2 * h]);
                    const long bv = (static_cast<long>(static_cast<std::uint32_t>(B[ni][2 * h + 1])) << 32) |
                                    static_cast<std::uint32_t>(B[ni][2 * h]);
                    if constexpr (!DBG) {
                        if constexpr (kBias) {
                            if constexpr (G == 32)
                                KQ_GASM("v_mfma_i32_16x16x32_i8 %0, %1, %2, %3" : "=&v"(c) : "v"(av), "v"(bv), "v"(biasv));
                            else
                                KQ_GASM("v_mfma_i32_16x16x64_i8 %0, %1, %2, %3" : "=&v"(c) : "v"(A[mi]), "v"(B[ni]), "v"(biasv));
                            return;
                        }
                        if constexpr (G == 32) KQ_GASM("v_mfma_i32_16x16x32_i8 %0, %1, %2, 0" : "=&v"(c) : "v"(av), "v"(bv));
                        else KQ_GASM("v_mfma_i32_16x16x64_i8 %0, %1, %2, 0" : "=&v"(c) : "v"(A[mi]), "v"(B[ni]));
                        return;
                    }
                    if constexpr (G == 32) c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, zero, 0, 0, 0);
                    else c = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mi], B[ni], zero, 0, 0, 0);
                };
                auto epilogue = [&](int blk, const v4i& c) {
                    const int mi = blk >> 2, ni = blk & 3;
                    if constexpr (!DBG && kBias) {
                        float t[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) KQ_GASM("v_fma_f32 %0, %1, %2, %3" : "=v"(t[r]) : "v"(c[r]), "v"(sv4[ni]), "v"(nb4[ni]));
#pragma unroll
                        for (int r = 0; r < 4; ++r) KQ_GASM("v_fmac_f32 %0, %1, %2" : "+v"(acc[mi][ni][r]) : "v"(as4[mi][r]), "v"(t[r]));
                        (void)t;  // (the host pass compiles the assembly out)
                        return;
                    }
                    if constexpr (!DBG) {
                        float kk[4], t[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if constexpr (QM == QUANT_STATIC) kk[r] = sv4[ni];
                            else KQ_GASM("v_mul_f32 %0, %1, %2" : "=v"(kk[r]) : "v"(as4[mi][r]), "v"(sv4[ni]));
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) KQ_GASM("v_cvt_f32_i32 %0, %1" : "=v"(t[r]) : "v"(c[r]));
#pragma unroll
                        for (int r = 0; r < 4; ++r) KQ_GASM("v_fmac_f32 %0, %1, %2" : "+v"(acc[mi][ni][r]) : "v"(kk[r]), "v"(t[r]));
                        (void)kk;
                        (void)t;  // (the host pass compiles the assembly out)
                        return;
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = m0 + wm * WV::WR + mi * 16 + 4 * L + r;
                        const int nt = nb * kSlots + 4 * wn + ni, col = nt * kTileRows + nn;
                        const int b = k * GPS + gi;
                        if (a.dump && row < a.M && nt < a.n_tiles && col < a.N && b < a.groups)
                            a.dump[(static_cast<std::int64_t>(row) * a.N + col) * a.groups + b] = c[r];
                        if constexpr (kBias) {  // the biased form's arithmetic: t = s * P' rounded once, then fused
                            const float t = sv4[ni] * static_cast<float>(c[r]);
                            acc[mi][ni][r] = __builtin_fmaf(as4[mi][r], t, acc[mi][ni][r]);
                            continue;
                        }
                        const float scale = QM == QUANT_STATIC ? sv4[ni] : as4[mi][r] * sv4[ni];
                        acc[mi][ni][r] = __builtin_fmaf(scale, static_cast<float>(c[r]), acc[mi][ni][r]);
                    }
                };
                // Software pipeline: block blk's MFMA, then block blk - 1's epilogue. An int8 MFMA result needs 8
                // wait states before a VALU reads it (what the compiler inserts for the builtin) and the hazard
                // recognizer does not look into inline assembly, so the distances are kept here: from block 1 on
                // the previous epilogue (12 VALU, 8 when calibrated or biased, plus 2 wait states then) and the next block's
                // MFMA lie between an MFMA and its epilogue; block 0's epilogue and block 15's wait on s_nop.
                v4i cp;
                mfmas(0, cp);
#pragma unroll
                for (int blk = 1; blk < 4 * MI; ++blk) {
                    v4i cn;
                    mfmas(blk, cn);
                    if (blk == 1) KQ_GASM("s_nop 7");
                    else if (QM == QUANT_STATIC || kBias) KQ_GASM("s_nop 1");
                    epilogue(blk - 1, cp);
                    cp = cn;
                }
                KQ_GASM("s_nop 7\n\ts_nop 7");
                epilogue(4 * MI - 1, cp);
            }
        }
        if (more) {
            store((k + 1) & 1);  // the other stage: its last readers passed the previous barrier
            __syncthreads();
        }
    }

    // ---- output ----
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm * WV::WR + mi * 16 + 4 * L + r;
            if (row >= a.M) continue;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int nt = nb * kSlots + 4 * wn + ni, col = nt * kTileRows + nn;
                if (nt >= a.n_tiles || col >= a.N) continue;
                float v = acc[mi][ni][r];
                if (QM == QUANT_STATIC) v = v * a.input_scale;
                a.y[static_cast<std::int64_t>(row) * a.N + col] = calibrate_output(v, a.output_scale);
            }
        }
    }
}

// Row quantizer for the g = 32 / 64 GEMM: one lane per 32 columns of a row (a lane pair per group when g = 64, one
// DPP step reduces it). The arithmetic is the shared quantizer's (quant_block / quant_code: Kidi's dynamic
// symmetric form, hnsw_test.cpp:513-520, or the calibrated rint(x / input_scale)); codes go to [M_p][K] in the
// tiles' permuted order (column 32 h + 8 L + i of a 64-column block at 16 L + 8 h + i: four 8-byte pieces per lane),
// block scales (and, for the parity dump, code sums) to [K/g][M_p]. Rows M .. M_p - 1 get codes 0 and scale 0.
struct QgArgs {
    const void* x;
    int x_f32;
    int M, M_p, K, g;
    float input_scale;
    std::int8_t* q;
    float* scale_t;
    std::int32_t* sum_t;  // optional
};

template <int QM>
__global__ __launch_bounds__(256) void quantize_rows_g_kernel(QgArgs a) {
    const int units = a.K / 32;
    const std::int64_t t = static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const std::int64_t m = t / units;
    const int j = static_cast<int>(t - m * units);
    if (m >= a.M_p) return;  // whole lane pairs: units is even
    const bool live = m < a.M;
    float v[32];
    const std::int64_t e0 = m * a.K + 32 * j;
    if (live) {
        if (a.x_f32) {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + e0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 r = p[i];
                v[4 * i] = r.x;
                v[4 * i + 1] = r.y;
                v[4 * i + 2] = r.z;
                v[4 * i + 3] = r.w;
            }
        } else {
            const uint4* p = reinterpret_cast<const uint4*>(static_cast<const std::uint16_t*>(a.x) + e0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 r = p[i];
                const std::uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    v[8 * i + 2 * d] = __uint_as_float(w4[d] << 16);
                    v[8 * i + 2 * d + 1] = __uint_as_float(w4[d] & 0xFFFF0000u);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = 0.F;
    }
    float mx = 0.F, mn = 0.F;
    if constexpr (QM != QUANT_STATIC) {
#pragma unroll
        for (int i = 0; i < 32; ++i) quant_stat(QM, v[i], mx, mn);
        if (a.g == 64) mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0xB1, 0xF, 0xF, true)));
    }
    const QuantBlock qb = quant_block(QM, mx, mn, a.input_scale, live);
    const int blk = j >> 1, h = j & 1;
    std::int8_t* row = a.q + m * a.K + 64 * blk + 8 * h;
    int total = 0;
#pragma unroll
    for (int L = 0; L < 4; ++L) {
        std::uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = live ? quant_code(QM, v[8 * L + i], qb, a.input_scale) : 0;
            total += c;
            if (i < 4) lo |= (static_cast<std::uint32_t>(c) & 0xFFu) << (8 * i);
            else hi |= (static_cast<std::uint32_t>(c) & 0xFFu) << (8 * (i - 4));
        }
        *reinterpret_cast<uint2*>(row + 16 * L) = make_uint2(lo, hi);
    }
    if (a.g == 64) total += __builtin_amdgcn_mov_dpp(total, 0xB1, 0xF, 0xF, true);
    if (a.g == 32 || h == 0) {
        const std::int64_t o = static_cast<std::int64_t>(a.g == 32 ? j : j >> 1) * a.M_p + m;
        a.scale_t[o] = qb.s;
        if (a.sum_t) a.sum_t[o] = total;
    }
}

// Parity dump: natural-order codes and [M][K/g] block statistics from the quantizer's outputs.
__global__ __launch_bounds__(256) void unpermute_g_kernel(const std::int8_t* q, int M, int K, std::int8_t* codes) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= static_cast<std::int64_t>(M) * K) return;
    const std::int64_t m = id / K, k = id % K;
    codes[id] = q[m * K + act_position(k)];
}
__global__ __launch_bounds__(256) void stats_g_kernel(const float* s_t, const std::int32_t* q_t, int M, int M_p, int groups,
                                                      float* s, std::int32_t* q, std::int32_t* z) {
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= static_cast<std::int64_t>(M) * groups) return;
    const std::int64_t m = id / groups, b = id % groups;
    if (s) s[id] = s_t[b * M_p + m];
    if (q) q[id] = q_t[b * M_p + m];
    if (z) z[id] = 0;
}

hipError_t launch_quantize_g(const LinearCall& c, std::int32_t* sums, hipStream_t stream) {
    const Weight& w = *c.w;
    QgArgs q{};
    q.x = c.x;
    q.x_f32 = c.x_type == ACT_F32;
    q.M = static_cast<int>(c.M);
    q.M_p = static_cast<int>(c.act.rows_p);
    q.K = static_cast<int>(w.geo.cols);
    q.g = w.geo.group;
    q.input_scale = c.input_scale;
    q.q = c.act.q;
    q.scale_t = c.act.scale;
    q.sum_t = sums;
    const std::int64_t lanes = static_cast<std::int64_t>(q.M_p) * (q.K / 32);
    const dim3 grid(static_cast<unsigned>((lanes + 255) / 256)), block(256);
    if (c.path == PATH_SYMMETRIC) hipLaunchKernelGGL((quantize_rows_g_kernel<QUANT_STATIC>), grid, block, 0, stream, q);
    else hipLaunchKernelGGL((quantize_rows_g_kernel<QUANT_DYN_SYM>), grid, block, 0, stream, q);
    return hipGetLastError();
}

}  // namespace

bool gemm_i4g_fits(const LinearCall& c) {
    const Weight& w = *c.w;
    if (!w.tiled || w.geo.bits != 4 || (w.geo.group != 32 && w.geo.group != 64) || c.M <= 16 || c.gelu_gate) return false;
    if (c.path != PATH_BLOCKWISE && c.path != PATH_SYMMETRIC) return false;
    if (w.zero_mode == ZERO_FLOAT) return false;
    if (w.geo.cols % kBK || w.geo.cols_p != w.geo.cols) return false;
    if (reinterpret_cast<std::uintptr_t>(c.x) & 15u) return false;  // the row quantizer's 16-byte loads
    const std::int64_t M_p = c.act.rows_p ? c.act.rows_p : round_up(c.M, 256);
    if (M_p % kBM || M_p * w.geo.cols >= (std::int64_t{1} << 31) || M_p * w.geo.groups_p >= (std::int64_t{1} << 31) ||
        w.geo.n_tiles * w.geo.k_tiles * kTileBytes >= (std::int64_t{1} << 46) || c.M * w.geo.rows >= (std::int64_t{1} << 31) ||
        (c.dump && c.M * w.geo.rows * (w.geo.cols / w.geo.group) >= (std::int64_t{1} << 62)))
        return false;
    return true;
}

hipError_t launch_gemm_i4g(const LinearCall& c, hipStream_t stream) {
    const Weight& w = *c.w;
    hipError_t e = launch_quantize_g(c, nullptr, stream);  // codes [rows_p][K] permuted, block scales [groups][rows_p]
    if (e != hipSuccess) return e;
    GArgs a{};
    a.q = c.act.q;
    a.a_scale = c.act.scale;
    a.tiles = w.tiles;
    a.scales = w.scales;
    a.zero_points = w.zero_mode == ZERO_POINT ? w.zero_points : nullptr;
    a.y = c.y;
    a.dump = c.dump;
    a.M = static_cast<int>(c.M);
    a.M_p = static_cast<int>(c.act.rows_p);
    a.N = static_cast<int>(w.geo.rows);
    a.K = static_cast<int>(w.geo.cols);
    a.k_tiles = static_cast<int>(w.geo.k_tiles);
    a.n_tiles = static_cast<int>(w.geo.n_tiles);
    a.groups_p = static_cast<int>(w.geo.groups_p);
    a.groups = static_cast<int>(w.geo.cols / w.geo.group);
    a.input_scale = c.input_scale;
    a.output_scale = c.output_scale;
    a.m_blocks = static_cast<int>((c.M + kBM - 1) / kBM);
    a.n_blocks = static_cast<int>((w.geo.n_tiles + kSlots - 1) / kSlots);
    if (a.m_blocks * kBM > a.M_p) return hipErrorInvalidValue;  // the activation panel must cover every tile row
    const dim3 grid(static_cast<unsigned>(a.m_blocks * a.n_blocks)), block(64 * kWaves);
    const bool stat = c.path == PATH_SYMMETRIC, zp = w.zero_mode == ZERO_POINT, sh = w.scale_type == META_F16;
    const bool dbg = c.dump != nullptr;
#define KQ_GG(G, QM, Z, H, D) hipLaunchKernelGGL((gemm_i4g_kernel<G, QM, Z, H, D, kWaves>), grid, block, GShape<G>::LDS, stream, a)
#define KQ_GGD(G, QM, Z, H) \
    if (dbg) KQ_GG(G, QM, Z, H, true); \
    else KQ_GG(G, QM, Z, H, false)
#define KQ_GGH(G, QM, Z) \
    if (sh) { KQ_GGD(G, QM, Z, true); } \
    else { KQ_GGD(G, QM, Z, false); }
#define KQ_GGQ(G)                                      \
    if (stat) { KQ_GGH(G, dev::QUANT_STATIC, false) } \
    else if (zp) { KQ_GGH(G, dev::QUANT_DYN_SYM, true) } \
    else { KQ_GGH(G, dev::QUANT_DYN_SYM, false) }
    if (w.geo.group == 32) { KQ_GGQ(32) }
    else { KQ_GGQ(64) }
#undef KQ_GGQ
#undef KQ_GGH
#undef KQ_GGD
#undef KQ_GG
    return hipGetLastError();
}

hipError_t launch_gemm_i4g_quantize_dump(const LinearCall& c, std::int8_t* codes, float* scales, std::int32_t* sums,
                                         std::int32_t* zero_points, hipStream_t stream) {
    hipError_t e = launch_quantize_g(c, c.act.sum, stream);
    if (e != hipSuccess) return e;
    const int M = static_cast<int>(c.M), K = static_cast<int>(c.w->geo.cols), groups = K / c.w->geo.group;
    const std::int64_t total = static_cast<std::int64_t>(M) * K;
    if (codes) hipLaunchKernelGGL(unpermute_g_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, c.act.q, M, K, codes);
    const std::int64_t st = static_cast<std::int64_t>(M) * groups;
    hipLaunchKernelGGL(stats_g_kernel, dim3(static_cast<unsigned>((st + 255) / 256)), dim3(256), 0, stream, c.act.scale, c.act.sum, M,
                       static_cast<int>(c.act.rows_p), groups, scales, sums, zero_points);
    return hipGetLastError();
}

}  // namespace kq
