// Prefill projection (M > 16) of the MI355X quantized linear layer for 4-bit weights with g = 128 on
// v_mfma_i32_32x32x32_i8, from a prefill copy of the weight.
//
// Prefill copy (built once when the weight is packed, kq_api.cpp build_prefill): the codes as int8 with the zero point
// folded in (u - zp for uint4 zero points, c otherwise), in the operand order of v_mfma_i32_32x32x32_i8: for each 32
// output columns and 32 input columns one 1 KiB fragment [64 lanes][16 B], lane l = column l % 32 and k-half
// h = l / 32, byte p holding k = 8 h + p (p < 8) or 16 + 8 h + p - 8; fragments of one column block are contiguous
// along K. Per (column, group) a record {s, -1.5 * 2^23 * s, z, 0}.
//
// quantize_rows8_kernel: one wave per 32 rows and one group: each lane reads the 16 columns of its fragment slot in
//   each of the group's four fragments (A operand: lane l = row l % 32), the two halves of a row combine their max |x|
//   across lanes l, l ^ 32, and every fragment leaves as one coalesced 1 KiB store; block scales transposed
//   [groups][M_p] in natural row order (and a_s * Q for additive zeros).
// gemm8_kernel: workgroup tile 256 rows x 128 columns, 8 waves of 64 x 64 (two 32-row blocks x two 32-column
//   blocks, two waves per SIMD), one 128-column k step (one group) per iteration. Operands and per-step metadata
//   (weight records, activation scales) reach LDS through direct copies only (buffer_load ... lds, 16 B per lane,
//   exactly 7 per wave and step) into a 3-stage ring of 52 KiB stages; each wave reads its fragments with
//   ds_read_b128 one block ahead of use. Per 32 x 32 block and group: four MFMAs whose first one
//   starts from the bits of 1.5 * 2^23, so the int32 result read as f32 is 12582912 + P' exactly (|P'| < 2^22); then
//   per element t = fma(bits, s, -12582912 s) = fl(s * P') (exact for F16-derived s) and acc += a_s * t, with a_s
//   broadcast from one register by DPP row_newbcast (the 16 rows a lane holds are lane-index-addressable in every
//   16-lane row). The epilogue of a block runs after MFMAs 2-4 of the next block (12 wait states after its last
//   MFMA), so its VALU issues in the shadow of the 8-pass MFMAs.
// Numerics: BlockwiseLinear / SymmetricPackedLinear closed forms (runtime/ynn/operators.cpp:1118-1169, :1250-1308),
// zero point folded into the integer operand, additive float zeros as acc += (a_s * Q) * z.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "kq_device.hpp"
#include "kq_internal.hpp"

namespace kq {
namespace {

using namespace dev;

typedef __attribute__((address_space(3))) void lds_void;
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));  // fp32 accumulators of a 32 x 32 block (the MFMA output layout)
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int kBM = 256;  // rows of the activation row padding (M_p) and of the wide tile (columns: 4 blocks of 32)
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr float kBias = 12582912.F;                  // 1.5 * 2^23
constexpr int kBiasBits = 0x4B400000;

// Step geometry of the GEMM for weight group size G and RB 32-row blocks per wave (tile rows TM = 128 RB). One k step
// is 128 columns (one group) for G = 128 and 64 columns (one group of 64 or two of 32) otherwise. One LDS stage (one k
// step): activation fragments [4 RB row blocks][CH k-chunks][1 KiB], weight fragments [4 column blocks][CH][1 KiB], the
// tile's activation scales [GPS groups][256 rows], a_s * Q (additive zeros) likewise, and the weight records [GPS][4
// column blocks][32 columns][16 B]. After the stages, 1 KiB that dummy copies write into. Direct copies per wave and
// step: RB CH / 2 activation fragments, CH / 2 weight fragments, one metadata block (or a dummy).
template <int G, int RB = 2>
struct Geo8 {
    static constexpr int TM = 128 * RB;
    static constexpr int kStepK = G == 128 ? 128 : 64;
    static constexpr int CH = kStepK / 32;           // 32-column chunks per step
    static constexpr int GPS = kStepK / G;           // groups per step
    static constexpr int kAOff = 0;
    static constexpr int kBOff = kAOff + 4 * RB * CH * 1024;
    static constexpr int kSOff = kBOff + 4 * CH * 1024;
    static constexpr int kZOff = kSOff + GPS * 1024;
    static constexpr int kWOff = kZOff + GPS * 1024;
    static constexpr int kStageBytes = kWOff + GPS * 2048;
    static constexpr int kStages = (G == 128 && RB == 2) ? 3 : 4;
    static constexpr int kDummyOff = kStages * kStageBytes;
    static constexpr int kLds = kDummyOff + 1024;  // RB = 2: G = 128: 157 KiB; 64: 113 KiB; 32: 129 KiB. RB = 1, G = 128: 145 KiB
    static constexpr int kACopies = RB * CH / 2;
    static constexpr int kCopies = kACopies + CH / 2 + 1;
    static_assert(kLds <= 160 * 1024, "LDS budget");
    static_assert(4 * GPS <= kWaves, "one metadata copy per wave");
};

#if defined(__HIP_DEVICE_COMPILE__)
#define KQ_ASM(...) asm volatile(__VA_ARGS__)
#else
#define KQ_ASM(...) (void)0
#endif

__device__ __forceinline__ std::uint32_t lds_addr(void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>((lds_void*)p));
#else
    return static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>(p));
#endif
}
template <int OFF>
__device__ __forceinline__ void ds_read16(v4i& v, std::uint32_t addr) {
    KQ_ASM("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
}
template <typename T>
__device__ __forceinline__ void tie(T& x) {
    KQ_ASM("" : "+v"(x));
}
template <typename T, int N>
__device__ __forceinline__ void tie(T (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) tie(x[i]);
}
// s_waitcnt lgkmcnt(N) that every guarded register depends on (no use can move above it)
template <int N, typename... T>
__device__ __forceinline__ void lgkm_wait(T&... x) {
    KQ_ASM("s_waitcnt lgkmcnt(%0)" : : "n"(N));
    (tie(x), ...);
}

constexpr int kRsrcWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kRsrcWord3);
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

// ------------------------------------------------------------------------------------------------------------------
// Row quantizer

// Byte position (lane half h, byte p) of column kk (0..31) of a 32-column chunk in the fragment order.
// kk 0..7 -> (0, kk), 8..15 -> (1, kk - 8), 16..23 -> (0, 8 + kk - 16), 24..31 -> (1, 8 + kk - 24)

struct QRow8Args {
    const void* x;
    int M, M_p, K;
    float input_scale;
    std::int8_t* q;         // [M_p/32][K/32][64][16]
    float* scale_t;         // [K/G][M_p] (dynamic)
    float* az_t;            // [K/G][M_p] a_s * Q (additive float zeros), or null
    const float* ninv;      // NORM: per-row inverse RMS [M]
    const float* nw;        // NORM: norm weight [K]
    // parity dumps (natural order), or null
    std::int8_t* d_codes;   // [M][K]
    float* d_scales;        // [M][K/G]
    std::int32_t* d_sums;   // [M][K/G]
};

// One wave per (32-row block, 128-column chunk): lane l = row l % 32, fragment half h = l / 32. For each of the
// chunk's four 32-column fragments f the lane reads its two 8-column pieces (columns 32 f + 8 h + 0..7 and
// 32 f + 16 + 8 h + 0..7), so its 16 code bytes are exactly its 16-byte slot of the fragment and each fragment is
// written as one coalesced 1 KiB store. Activation blocks are the weight's groups (G = 32, 64 or 128 columns: one, two
// or four fragments); a row's max |x| over a block combines the two halves through lane l ^ 32.
template <int QM, bool F32, bool NORM, int G>
__global__ __launch_bounds__(256) void quantize_rows8_kernel(QRow8Args a) {
    constexpr int NBLK = 128 / G, FPB = G / 32;  // blocks per chunk, fragments per block
    const int chunks = a.K / 128, KC = a.K / 32, groups = a.K / G;
    const int item = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
    if (item >= (a.M_p / 32) * chunks) return;  // whole waves
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int mb = item / chunks, g = item - mb * chunks;
    const int r = lane & 31, h = lane >> 5;
    const int m = 32 * mb + r;
    const bool live = m < a.M;
    // v[8 f + 4 p + ...]: piece p (0: columns 32 f + 8 h + 0..7, 1: 32 f + 16 + 8 h + 0..7) of fragment f
    float v[64];
    const int c0 = 128 * g + 8 * h;
    if (live) {
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
            for (int pc = 0; pc < 2; ++pc) {
                const int col = c0 + 32 * f + 16 * pc;
                float* d = v + 16 * f + 8 * pc;
                if constexpr (F32) {
                    const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + static_cast<std::int64_t>(m) * a.K + col);
                    const float4 r0 = src[0], r1 = src[1];
                    d[0] = r0.x; d[1] = r0.y; d[2] = r0.z; d[3] = r0.w;
                    d[4] = r1.x; d[5] = r1.y; d[6] = r1.z; d[7] = r1.w;
                } else {
                    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const std::uint16_t*>(a.x) + static_cast<std::int64_t>(m) * a.K + col);
                    const std::uint32_t w4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        d[2 * e] = __uint_as_float(w4[e] << 16);
                        d[2 * e + 1] = __uint_as_float(w4[e] & 0xFFFF0000u);
                    }
                }
                if constexpr (NORM) {
                    const float inv = a.ninv[m];
                    const float4* wp = reinterpret_cast<const float4*>(a.nw + col);
                    const float4 n0 = wp[0], n1 = wp[1];
                    const float nw[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) d[e] = d[e] * inv * nw[e];
                }
            }
    } else {
#pragma unroll
        for (int i = 0; i < 64; ++i) v[i] = 0.F;
    }
    QuantBlock qbs[NBLK];
#pragma unroll
    for (int bb = 0; bb < NBLK; ++bb) {
        float mx = 0.F, mn = 0.F;
        if constexpr (QM != QUANT_STATIC) {
#pragma unroll
            for (int i = 16 * FPB * bb; i < 16 * FPB * (bb + 1); ++i) quant_stat(QM, v[i], mx, mn);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
        }
        qbs[bb] = quant_block(QM, mx, mn, a.input_scale, live);
    }
    // codes: w[4 f + i] holds the lane's bytes 4 i .. 4 i + 3 of fragment f (its 16-byte slot)
    std::uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const QuantBlock& qb = qbs[i / (4 * FPB)];
        if constexpr (QM == QUANT_STATIC) {
            std::uint32_t d = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float c = fminf(fmaxf(__builtin_rintf(v[4 * i + e] / a.input_scale), -128.F), 127.F);
                d = __builtin_amdgcn_cvt_pk_u8_f32(c + 128.F, e, d);
            }
            w[i] = d ^ 0x80808080u;
        } else {
            // dynamic: |x * inverse| <= 127 (1 + 2^-24) rounds to at most 127 (no clamp); adding 1.5 * 2^23 rounds
            // x * inverse to the nearest integer (ties to even, as rint), held in the low mantissa byte
            std::uint32_t u[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) u[e] = __float_as_uint(v[4 * i + e] * qb.inverse + kBias);
            const std::uint32_t lo = __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0400u), hi = __builtin_amdgcn_perm(u[3], u[2], 0x0c0c0400u);
            w[i] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
    }
    std::int8_t* frag = a.q + (static_cast<std::int64_t>(mb) * KC + 4 * g) * 1024 + lane * 16;
#pragma unroll
    for (int f = 0; f < 4; ++f)
        *reinterpret_cast<uint4*>(frag + f * 1024) = make_uint4(w[4 * f], w[4 * f + 1], w[4 * f + 2], w[4 * f + 3]);
    // per block: code sums (additive float zeros and the parity dump), scales
#pragma unroll
    for (int bb = 0; bb < NBLK; ++bb) {
        int qsum = 0;
        if (a.az_t || a.d_sums) {
#pragma unroll
            for (int i = 4 * FPB * bb; i < 4 * FPB * (bb + 1); ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) qsum += static_cast<std::int8_t>((w[i] >> (8 * e)) & 0xFFu);
            qsum += __shfl_xor(qsum, 32);
        }
        if (h == 0) {
            const int gb = NBLK * g + bb;  // the block's group index
            const std::int64_t o = static_cast<std::int64_t>(gb) * a.M_p + m;
            if (a.scale_t) a.scale_t[o] = qbs[bb].s;
            if (a.az_t) a.az_t[o] = qbs[bb].s * static_cast<float>(qsum);
            if (live && a.d_scales) a.d_scales[static_cast<std::int64_t>(m) * groups + gb] = QM == QUANT_STATIC ? a.input_scale : qbs[bb].s;
            if (live && a.d_sums) a.d_sums[static_cast<std::int64_t>(m) * groups + gb] = qsum;
        }
    }
    if (live && a.d_codes) {
        // natural column order: piece p of fragment f holds columns 32 f + 16 p + 8 h + 0..7
        std::int8_t* dst = a.d_codes + static_cast<std::int64_t>(m) * a.K + c0;
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
            for (int pc = 0; pc < 2; ++pc)
                *reinterpret_cast<uint2*>(dst + 32 * f + 16 * pc) = make_uint2(w[4 * f + 2 * pc], w[4 * f + 2 * pc + 1]);
    }
}


// ------------------------------------------------------------------------------------------------------------------
// GEMM

struct Gemm8Args {
    const std::int8_t* q;       // activation fragments [M_p/32][K/32][64][16]
    const float* scale_t;       // [groups][M_p] activation block scales (dynamic)
    const float* az_t;          // [groups][M_p] a_s * Q (additive float zeros)
    const std::int8_t* w;       // weight fragments [NB][K/32][64][16]
    const float4* wmeta;        // [groups][NB][32] {s, -1.5 * 2^23 * s, z, 0}
    float* y;
    std::int32_t* dump;         // [M][N][groups] P' (parity instrumentation), or null
    float* partial;             // split K: [ksplit][tiles][512 threads][64] raw accumulators
    int M, M_p, N, K, NB, groups, m_blocks, n_blocks, ksplit;
    float input_scale, output_scale;
};

// Global 32-column block of workgroup column block nb, local block cb (0..3); >= NB when out of range. GELU: cb 0, 1
// are gate blocks 2 nb + cb, cb 2, 3 the matching up blocks (gate rows [0, I), up rows [I, 2I), I a multiple of 32).
template <bool GELU>
__device__ __forceinline__ int col_block(const Gemm8Args& a, int nb, int cb) {
    if constexpr (GELU) {
        const int half = a.NB >> 1;
        const int g = 2 * nb + (cb & 1);
        return g < half ? (cb < 2 ? g : half + g) : a.NB;
    }
    return 4 * nb + cb;
}

// Row (within its 32-row block) of element k (0..15) of a 32 x 32 result held by lane l: 8 (k / 4) + 4 (l / 32) + k % 4.
// The DPP broadcast register of a row block holds, at lane 16 r + k, the value of that row for lanes of row r.
__device__ __forceinline__ int bcast_row(int lane) { return 8 * ((lane & 15) >> 2) + 4 * (lane >> 5) + (lane & 3); }

template <int GPS>
struct Meta {  // one k step's epilogue operands of a wave: weight records of its two column blocks, scales of its rows
    v2i rec[2][GPS];   // {s, -1.5 * 2^23 * s} of the lane's column in column blocks 0, 1, per group of the step
    float z[2][GPS];   // its additive zero z (additive zeros)
    float as[2][GPS];  // a_s of DPP row bcast_row(lane) in row blocks 0, 1
    float az[2][GPS];  // a_s * Q likewise (additive zeros)
};

// Epilogue of elements [K0, K1) of one block; P holds the biased int32 partials (as f32: 12582912 + P'). Each slice
// issues its conversions first and its accumulations after, so no accumulation reads a register written by the
// instruction right before it.
//   F16 scales, dynamic:    P = fma(P, s, nb) = fl(s * P');   acc += a_s[row] * P   (a_s broadcast by DPP)
//   F16 scales, calibrated: P = fma(P, s, nb);                 acc += P (input_scale applied at the end)
//   F32 scales, dynamic:    P = P - 12582912 (exact);  P = P * s;  acc += a_s[row] * P
//   F32 scales, calibrated: P = P - 12582912;          acc += P * s
//   additive zeros:         acc += (a_s * Q)[row] * z
template <int K, bool SF16, bool STAT>
__device__ __forceinline__ void epi_convert(int& P, const v2i& rec) {
    if constexpr (SF16) {
        KQ_ASM("v_fma_f32 %0, %0, %1, %2" : "+v"(P) : "v"(rec[0]), "v"(rec[1]));
    } else {
        KQ_ASM("v_add_f32 %0, 0xcb400000, %0" : "+v"(P));
        if constexpr (!STAT) KQ_ASM("v_mul_f32 %0, %0, %1" : "+v"(P) : "v"(rec[0]));
    }
}
template <int K, bool SF16, bool STAT, bool ZF>
__device__ __forceinline__ void epi_accumulate(float& acc, int P, const v2i& rec, float z, float as, float az) {
    if constexpr (STAT) {
        if constexpr (SF16) KQ_ASM("v_add_f32 %0, %0, %1" : "+v"(acc) : "v"(P));
        else KQ_ASM("v_fmac_f32 %0, %1, %2" : "+v"(acc) : "v"(P), "v"(rec[0]));
    } else {
        KQ_ASM("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(as), "v"(P), "n"(K));
    }
    if constexpr (ZF)
        KQ_ASM("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(az), "v"(z), "n"(K));
}
template <int K0, int K1, bool SF16, bool STAT>
__device__ __forceinline__ void epi_converts(v16i& P, const v2i& rec) {
    if constexpr (K0 < K1) {
        int p = P[K0];
        epi_convert<K0, SF16, STAT>(p, rec);
        P[K0] = p;
        epi_converts<K0 + 1, K1, SF16, STAT>(P, rec);
    }
}
// (AccT: float[16], or v16f where an MFMA also accumulates into the block and needs it as one register tuple)
template <int K0, int K1, bool SF16, bool STAT, bool ZF, typename AccT>
__device__ __forceinline__ void epi_accumulates(AccT& acc, const v16i& P, const v2i& rec, float z, float as, float az) {
    if constexpr (K0 < K1) {
        float x = acc[K0];
        epi_accumulate<K0, SF16, STAT, ZF>(x, P[K0], rec, z, as, az);
        acc[K0] = x;
        epi_accumulates<K0 + 1, K1, SF16, STAT, ZF>(acc, P, rec, z, as, az);
    }
}
// DBG first stores P' = P - 0x4B400000 to the dump through a buffer resource: element k of the block is at byte
// voff + (8 (k / 4) + k % 4) N G 4 + g 4; lanes of columns past N carry an offset beyond the buffer, and rows past M
// land beyond it too, so the hardware drops those stores.
template <int K0, int K1, bool DBG>
__device__ __forceinline__ void epi_dump(const v16i& P, __amdgpu_buffer_rsrc_t dres, std::uint32_t voff, std::uint32_t row_bytes,
                                         std::uint32_t g_bytes) {
    if constexpr (DBG && K0 < K1) {
        int v = 0;  // (inline assembly keeps this read of the MFMA result in the epilogue's place)
        KQ_ASM("v_subrev_u32 %0, %1, %2" : "=v"(v) : "v"(kBiasBits), "v"(P[K0]));
        __builtin_amdgcn_raw_buffer_store_b32(v, dres, voff, (8 * (K0 >> 2) + (K0 & 3)) * row_bytes + g_bytes, 0);
        epi_dump<K0 + 1, K1, DBG>(P, dres, voff, row_bytes, g_bytes);
    }
}
struct Dump {
    const std::int32_t* base;  // the tile's first row
    std::uint32_t bytes;       // the buffer's extent from base
    std::uint32_t row_bytes;   // N * groups * 4
};
template <int K0, int K1, bool SF16, bool STAT, bool ZF, bool DBG, typename AccT>
__device__ __forceinline__ void epi_range(AccT& acc, v16i& P, const v2i& rec, float z, float as, float az, const Dump& d,
                                          std::uint32_t voff, int g) {
    if constexpr (DBG) epi_dump<K0, K1, DBG>(P, rsrc(d.base, d.bytes), voff, d.row_bytes, static_cast<std::uint32_t>(g) * 4);
    epi_converts<K0, K1, SF16, STAT>(P, rec);
    epi_accumulates<K0, K1, SF16, STAT, ZF>(acc, P, rec, z, as, az);
}

__device__ __forceinline__ void mfma_first(v16i& P, const v4i& A, const v4i& B, const v16i& bias) {
    KQ_ASM("v_mfma_i32_32x32x32_i8 %0, %1, %2, %3" : "=&v"(P) : "v"(A), "v"(B), "v"(bias));
}
__device__ __forceinline__ void mfma_acc(v16i& P, const v4i& A, const v4i& B) {
    KQ_ASM("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(P) : "v"(A), "v"(B));
}
// Additive float zeros of a block and a pair of groups (g, g + 1) straight into its fp32 accumulators:
// acc[row][col] += a[row][0] b[0][col] + a[row][1] b[1][col] with a[row][k] = (a_s * Q)[row, g + k] (lane l: row
// l % 32, k = l / 32) and b[k][col] = z[g + k, col] (lane l: column l % 32, k = l / 32); the result layout is the
// 32 x 32 layout of the int8 MFMAs. The two wait states cover VALU writes of acc, a and b just before it.
__device__ __forceinline__ void mfma_zero(v16f& acc, float a, float b) {
    KQ_ASM("s_nop 1\n\tv_mfma_f32_32x32x2_f32 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}

// 4 x 4 transpose inside each lane quad: on entry lane q of the quad holds v[e] = element (row e, column q); on exit
// v[e] = element (row q, column e). Two butterfly rounds of quad_perm DPP moves and lane-parity selects.
__device__ __forceinline__ void quad_transpose(float (&v)[4], int lane) {
    const bool b0 = lane & 1, b1 = lane & 2;
    const int x0 = __float_as_int(v[0]), x1 = __float_as_int(v[1]), x2 = __float_as_int(v[2]), x3 = __float_as_int(v[3]);
    const int s0 = dpp<0xB1>(x1), s1 = dpp<0xB1>(x0), s2 = dpp<0xB1>(x3), s3 = dpp<0xB1>(x2);  // lanes q ^ 1
    const int u0 = b0 ? s0 : x0, u1 = b0 ? x1 : s1, u2 = b0 ? s2 : x2, u3 = b0 ? x3 : s3;
    const int t0 = dpp<0x4E>(u2), t1 = dpp<0x4E>(u3), t2 = dpp<0x4E>(u0), t3 = dpp<0x4E>(u1);  // lanes q ^ 2
    v[0] = __int_as_float(b1 ? t0 : u0);
    v[1] = __int_as_float(b1 ? t1 : u1);
    v[2] = __int_as_float(b1 ? u2 : t2);
    v[3] = __int_as_float(b1 ? u3 : t3);
}

// Final values of a wave's 2 x 2 blocks (calibrated inputs scale by input_scale, calibrated outputs round to
// output_scale steps, GELU pairs column block 0 (gate) with 1 (up)), stored with 16-byte stores: each 4 x 4 sub-block
// (rows 8 j + 4 h + 0..3, four columns of a lane quad) is transposed in the quad, so lane q writes row 8 j + 4 h + q,
// columns 4 (col / 4) .. + 3. Every lane issues exactly 16 (GELU: kTileStoresGelu) stores; rows past M and columns
// past N fall outside the buffer resource, whose range check drops them, so the number of outstanding vector memory
// operations after a tile is known at compile time. (Plain projections use store8d below.)
constexpr int kTileStoresGelu = 8;
constexpr int min63(int n) { return n < 63 ? n : 63; }
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
template <bool STAT, bool GELU, int RB = 2, typename AccT>
__device__ __forceinline__ void store8t(const Gemm8Args& a, const AccT (&acc)[RB][2], int m0, int wm, const int (&gc)[2],
                                        int lane) {
    const int n_out = GELU ? (a.N >> 1) : a.N;
    const int rows = min(a.M - m0, 128 * RB);
    const __amdgpu_buffer_rsrc_t yres = rsrc(a.y + static_cast<std::int64_t>(m0) * n_out, static_cast<std::uint32_t>(rows) * n_out * 4);
    const int r_lane = 32 * RB * wm + 4 * (lane >> 5) + (lane & 3), c_lane = lane & 28;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const std::uint32_t row_off = static_cast<std::uint32_t>(r_lane + 32 * i + 8 * j) * n_out;
#pragma unroll
            for (int c = 0; c < (GELU ? 1 : 2); ++c) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 4 * j + e;
                    if constexpr (GELU) {
                        float g = acc[i][0][k], up = acc[i][1][k];
                        if (STAT) {
                            g = g * a.input_scale;
                            up = up * a.input_scale;
                        }
                        v[e] = gelu_tanh(calibrate_output(g, a.output_scale)) * calibrate_output(up, a.output_scale);
                    } else {
                        float x = acc[i][c][k];
                        if (STAT) x = x * a.input_scale;
                        v[e] = calibrate_output(x, a.output_scale);
                    }
                }
                quad_transpose(v, lane);
                const int n = 32 * gc[c] + c_lane;
                const bool live = GELU ? (gc[0] < (a.NB >> 1) && n < n_out) : n < n_out;
                const std::uint32_t voff = live ? (row_off + static_cast<std::uint32_t>(n)) * 4 : 0x80000000u;
                __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
                                                      yres, voff, 0, 0);
            }
        }
    }
}

// Final values of a wave's RB x 2 blocks for plain projections, stored straight from the accumulators with 4-byte
// stores (no transpose: every VALU instruction counts in this VALU-bound kernel). Element k of block (i, c) is row
// 32 RB wm + 32 i + 8 (k / 4) + 4 (lane / 32) + k % 4, column 32 gc[c] + lane % 32: one store instruction writes two
// 128-byte row segments. Every lane issues exactly 32 RB stores; rows past M and columns past N get a per-lane
// offset beyond the buffer resource, whose range check drops them.
template <bool STAT, int RB = 2, typename AccT>
__device__ __forceinline__ void store8d(const Gemm8Args& a, const AccT (&acc)[RB][2], int m0, int wm, const int (&gc)[2],
                                        int lane) {
    const int n_out = a.N;
    const int rows = min(a.M - m0, 128 * RB);
    const __amdgpu_buffer_rsrc_t yres = rsrc(a.y + static_cast<std::int64_t>(m0) * n_out, static_cast<std::uint32_t>(rows) * n_out * 4);
    const std::uint32_t row_bytes = static_cast<std::uint32_t>(n_out) * 4;
    const bool cal = a.output_scale > 0.F;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int n = 32 * gc[c] + (lane & 31);
        // dead columns: an offset past the buffer that stays past it for every row added below (rows * row_bytes < 2^31)
        const std::uint32_t col_off = n < n_out ? static_cast<std::uint32_t>(n) * 4 : 0x80000000u;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const std::uint32_t base = col_off + static_cast<std::uint32_t>(32 * RB * wm + 32 * i + 4 * (lane >> 5)) * row_bytes;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                float x = acc[i][c][k];
                if (STAT) x = x * a.input_scale;
                if (cal) x = calibrate_output(x, a.output_scale);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), yres,
                                                      base + static_cast<std::uint32_t>(8 * (k >> 2) + (k & 3)) * row_bytes, 0, 0);
            }
        }
    }
}

// One work item of gemm8_kernel: K range, tile, the tile's first row and its column block. (Declared at namespace
// scope: local classes in a kernel template keep the host pass from emitting the kernel's launch stub.)
struct Item {
    int ks, tile, m0, nbk;
};
// Copy parameters of one item and wave: the activation and weight sources, the weight extent, the metadata offset at
// the item's first k step, and that step.
struct Copy {
    const std::int8_t* abase;
    const std::int8_t* bbase;
    std::uint32_t bbytes, meta0;
    int kbase;
};

template <int G, int RB, bool SF16, bool STAT, bool ZF, bool GELU, bool SPLIT, bool DBG>
__global__ __launch_bounds__(kThreads) void gemm8_kernel(Gemm8Args a) {
    using Q = Geo8<G, RB>;
    constexpr int CH = Q::CH, GPS = Q::GPS, NS = Q::kStages, TM = Q::TM;
    static_assert(RB == 2 || (G == 128 && !GELU && !SPLIT), "the 128-row tile serves plain g = 128 projections without split K");
    // additive float zeros: on an fp32 MFMA per block and pair of steps in the 256 x 128 g = 128 body (ZM), else one
    // more VALU per element and group in the epilogue (ZFE)
    constexpr bool ZM = ZF && G == 128 && RB == 2;
    constexpr bool ZFE = ZF && !ZM;
    extern __shared__ __attribute__((aligned(16))) std::uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 3, wn = wave >> 2;  // rows [32 RB wm, +32 RB) of the tile; column blocks below
    const std::uint32_t lds0 = lds_addr(lds);

    // Work items (K range, row block, column block) in an order that gives each XCD a contiguous range of tiles, row
    // blocks fastest (the XCD's few column blocks of weights stay in its L2): item i of the launch is tile
    // (i % 8) (total / 8) + i / 8 when total % 8 == 0. The launch holds at most one workgroup per CU; workgroup b runs
    // items b, b + W, b + 2 W, ... (W workgroups) back to back, with the copy ring running on across item boundaries,
    // so the copies of an item's first steps are in flight during the previous item's last steps and its output
    // stores overlap the next item's MFMAs.
    const int tiles = a.m_blocks * a.n_blocks;
    const int total = tiles * a.ksplit;
    const int W = static_cast<int>(gridDim.x);
    const int bx = static_cast<int>(blockIdx.x);
    const int items = (total - bx + W - 1) / W;
    const int KC = a.K / 32;
    const int steps = a.K / Q::kStepK / a.ksplit;
    auto item_of = [&](int r) __attribute__((always_inline)) {
        int i = r * W + bx;
        if (total % 8 == 0) i = (i % 8) * (total / 8) + i / 8;
        Item it;
        it.ks = i / tiles;
        it.tile = i - it.ks * tiles;
        it.m0 = (it.tile % a.m_blocks) * TM;
        it.nbk = it.tile / a.m_blocks;
        return it;
    };

    // ---- copies of one step: wave w brings RB CH / 2 activation fragments (RB = 2: row block w; RB = 1: half of row
    // block w / 2), half of weight column block w / 2 (CH / 2 fragments) and one metadata block: waves 0 .. 2 GPS - 1 the weight records of group w / 2 of the step,
    // column blocks 0-1 (w even) or 2-3; the next GPS waves the tile's activation scales of one group each; the next
    // GPS its a_s * Q (additive zeros); the other copies write into the dummy area.
    const int cbc = wave >> 1, ckc = (CH / 2) * (wave & 1);
    // The wave's metadata copy: its resource, per-step stride and LDS place do not depend on the item (dummy: mdst < 0).
    // meta_gg: the offset of the wave's group within a step's metadata (0 when a step holds one group)
    __amdgpu_buffer_rsrc_t mres = rsrc(a.wmeta, 0u);
    std::uint32_t meta_step = 0, meta_gg = 0;
    int mdst = -1;
    if (wave < 2 * GPS) {
        const int mgg = GPS == 1 ? 0 : wave >> 1;
        mres = rsrc(a.wmeta, static_cast<std::uint32_t>(a.groups) * a.NB * 512);
        meta_step = static_cast<std::uint32_t>(GPS * a.NB) * 512;
        meta_gg = static_cast<std::uint32_t>(mgg * a.NB) * 512;
        mdst = Q::kWOff + mgg * 2048 + (wave & 1) * 1024;
    } else if ((wave < 3 * GPS && !STAT) || (wave >= 3 * GPS && wave < 4 * GPS && ZF)) {
        const bool sc = wave < 3 * GPS;
        const int mgg = GPS == 1 ? 0 : wave - (sc ? 2 : 3) * GPS;
        mres = rsrc(sc ? a.scale_t : a.az_t, static_cast<std::uint32_t>(a.groups) * a.M_p * 4);
        meta_step = static_cast<std::uint32_t>(GPS * a.M_p) * 4;
        meta_gg = static_cast<std::uint32_t>(mgg * a.M_p) * 4;
        mdst = (sc ? Q::kSOff : Q::kZOff) + mgg * 1024;
    }
    auto copy_of = [&](int r) __attribute__((always_inline)) {
        const Item it = item_of(r);
        Copy cp;
        cp.kbase = it.ks * steps;
        cp.abase = a.q + static_cast<std::int64_t>(it.m0 / 32) * KC * 1024;  // the tile's first row block
        const int gcb = col_block<GELU>(a, it.nbk, cbc);
        const bool clive = gcb < a.NB;
        cp.bbase = a.w + static_cast<std::int64_t>(clive ? gcb : 0) * KC * 1024;
        cp.bbytes = clive ? static_cast<std::uint32_t>(KC) * 1024 : 0u;
        cp.meta0 = 0x80000000u;
        if (wave < 2 * GPS)
            cp.meta0 = static_cast<std::uint32_t>(cp.kbase) * meta_step + meta_gg +
                       static_cast<std::uint32_t>(col_block<GELU>(a, it.nbk, 2 * (wave & 1))) * 512;
        else if (mdst >= 0)
            cp.meta0 = static_cast<std::uint32_t>(cp.kbase) * meta_step + meta_gg + static_cast<std::uint32_t>(it.m0) * 4;
        return cp;
    };
    // part 0: activation fragments [0, CH / 2) of the wave's row block (RB = 1: its half of the chunks), part 1 (RB =
    // 2): [CH / 2, CH), part 2: weight fragments and metadata
    const int arb = RB == 2 ? wave : wave >> 1, ack = RB == 2 ? 0 : (CH / 2) * (wave & 1);
    // st: byte offset of the target stage; kc0: the step's first 32-column chunk
    auto issue_copy = [&](const Copy& cp, std::uint32_t st, std::uint32_t kc0, int t, auto part) __attribute__((always_inline)) {
        constexpr int pt = decltype(part)::value;
        std::uint8_t* base = lds + st;
        if constexpr (pt < 2) {
            if constexpr (RB == 2 || pt == 0) {
                const __amdgpu_buffer_rsrc_t ares = rsrc(cp.abase, static_cast<std::uint32_t>(TM / 32) * KC * 1024);
#pragma unroll
                for (int i = ack + pt * (CH / 2); i < ack + (pt + 1) * (CH / 2); ++i)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lds_void*)(base + Q::kAOff + (arb * CH + i) * 1024), 16,
                                                             lane * 16, (static_cast<std::uint32_t>(arb) * KC + kc0 + i) * 1024, 0, 0);
            }
        } else {
            const __amdgpu_buffer_rsrc_t bres = rsrc(cp.bbase, cp.bbytes);
#pragma unroll
            for (int i = 0; i < CH / 2; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (lds_void*)(base + Q::kBOff + (cbc * CH + ckc + i) * 1024), 16,
                                                         lane * 16, (kc0 + ckc + i) * 1024, 0, 0);
            std::uint8_t* md = mdst < 0 ? lds + Q::kDummyOff : base + mdst;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_void*)md, 16, lane * 16, cp.meta0 + static_cast<std::uint32_t>(t) * meta_step, 0, 0);
        }
    };
    // issue(st, r, t): the copies of step t of item r into the stage at byte offset st; t may run past the item (the
    // next items' steps), and past the last item the item's last step is copied again, into a stage nothing reads any
    // more. item_copy holds the copy parameters of the item being computed. The scalar work is done once per step (not
    // per part), and the item-boundary path runs only in the last NS steps of an item.
    Copy item_copy = copy_of(0);
    auto issue_all = [&](const Copy& cp, std::uint32_t st, int t) __attribute__((always_inline)) {
        const std::uint32_t kc0 = static_cast<std::uint32_t>((cp.kbase + t) * CH);
        issue_copy(cp, st, kc0, t, std::integral_constant<int, 0>{});
        issue_copy(cp, st, kc0, t, std::integral_constant<int, 1>{});
        issue_copy(cp, st, kc0, t, std::integral_constant<int, 2>{});
    };
    auto issue = [&](std::uint32_t st, int r, int t) __attribute__((always_inline)) {
        if (t < steps) {
            issue_all(item_copy, st, t);
            return;
        }
        while (t >= steps) {
            t -= steps;
            ++r;
        }
        if (r >= items) issue_all(item_copy, st, steps - 1);
        else issue_all(copy_of(r), st, t);
    };

    // ---- the wave's fragments: row blocks RB wm + i; column blocks (plain) 2 wn + i, (GELU) wn + 2 i
    const int cb_l0 = GELU ? wn : 2 * wn, cb_l1 = GELU ? wn + 2 : 2 * wn + 1;
    const std::uint32_t a_lane = lds0 + Q::kAOff + (RB * wm * CH) * 1024 + lane * 16;
    const std::uint32_t b_lane0 = lds0 + Q::kBOff + (cb_l0 * CH) * 1024 + lane * 16;
    const std::uint32_t b_lane1 = lds0 + Q::kBOff + (cb_l1 * CH) * 1024 + lane * 16;
    const int col = lane & 31;
    [[maybe_unused]] const std::uint32_t w_lane0 = lds0 + Q::kWOff + (cb_l0 * 32 + col) * 16;
    [[maybe_unused]] const std::uint32_t w_lane1 = lds0 + Q::kWOff + (cb_l1 * 32 + col) * 16;
    [[maybe_unused]] const std::uint32_t s_lane = lds0 + Q::kSOff + (32 * RB * wm + bcast_row(lane)) * 4;
    // a_s * Q of row bcast_row(lane) (the epilogue's DPP broadcast), or of row lane % 32 (the MFMA's A operand)
    [[maybe_unused]] const std::uint32_t z_lane = lds0 + Q::kZOff + (32 * RB * wm + (ZM ? (lane & 31) : bcast_row(lane))) * 4;
    auto read_meta = [&](Meta<GPS>& mt, std::uint32_t stage) __attribute__((always_inline)) {
#pragma unroll
        for (int gg = 0; gg < GPS; ++gg) {
            KQ_ASM("ds_read_b64 %0, %1 offset:%2" : "=v"(mt.rec[0][gg]) : "v"(w_lane0 + stage), "n"(gg * 2048));
            KQ_ASM("ds_read_b64 %0, %1 offset:%2" : "=v"(mt.rec[1][gg]) : "v"(w_lane1 + stage), "n"(gg * 2048));
            if constexpr (ZF) {
                KQ_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(mt.z[0][gg]) : "v"(w_lane0 + stage), "n"(gg * 2048 + 8));
                KQ_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(mt.z[1][gg]) : "v"(w_lane1 + stage), "n"(gg * 2048 + 8));
            }
            if constexpr (!STAT) {
                KQ_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(mt.as[0][gg]) : "v"(s_lane + stage), "n"(gg * 1024));
                if constexpr (RB == 2)
                    KQ_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(mt.as[1][gg]) : "v"(s_lane + stage), "n"(gg * 1024 + 128));
            }
            if constexpr (ZF) {
                KQ_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(mt.az[0][gg]) : "v"(z_lane + stage), "n"(gg * 1024));
                if constexpr (RB == 2)
                    KQ_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(mt.az[1][gg]) : "v"(z_lane + stage), "n"(gg * 1024 + 128));
            }
        }
    };
    auto read_frags = [&](v4i (&f)[CH], std::uint32_t addr) __attribute__((always_inline)) {
        ds_read16<0>(f[0], addr);
        ds_read16<1024>(f[1], addr);
        if constexpr (CH == 4) {
            ds_read16<2048>(f[2], addr);
            ds_read16<3072>(f[3], addr);
        }
    };

    // ---- per item: the wave's global column blocks, the tile's first row, and the parity dump's resource and offsets
    // (DBG: P' of element (row, column n, group g) at dump[(row N + n) G + g]; dvo[i][c] is the byte offset of the lane's
    // element 0 in block (i, c), beyond the buffer for columns past N)
    int gc[2] = {0, 0};
    int m0 = 0, ks = 0, tile = 0;
    Dump dmp{};
    std::uint32_t dvo[RB][2] = {};
    auto begin_item = [&](int r) __attribute__((always_inline)) {
        const Item it = item_of(r);
        if (r > 0) item_copy = copy_of(r);
        m0 = it.m0;
        ks = it.ks;
        tile = it.tile;
        gc[0] = col_block<GELU>(a, it.nbk, cb_l0);
        gc[1] = col_block<GELU>(a, it.nbk, cb_l1);
        if constexpr (DBG) {
            // the resource starts at the tile's first row, so every offset stays far below 2^31
            const std::uint64_t row_elems = static_cast<std::uint64_t>(a.N) * a.groups;
            const std::uint64_t rest = static_cast<std::uint64_t>(a.M - m0) * row_elems * 4;
            dmp.base = a.dump + static_cast<std::uint64_t>(m0) * row_elems;
            dmp.bytes = static_cast<std::uint32_t>(rest < 0x7FFFFFFFull ? rest : 0x7FFFFFFFull);
            dmp.row_bytes = static_cast<std::uint32_t>(row_elems * 4);
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int n = 32 * gc[c] + col, r0 = 32 * RB * wm + 32 * i + 4 * (lane >> 5);
                    dvo[i][c] = (gc[c] < a.NB && n < a.N && m0 + r0 < a.M)
                                    ? static_cast<std::uint32_t>((static_cast<std::uint64_t>(r0) * a.N + n) * a.groups * 4)
                                    : 0x80000000u;
                }
        }
    };
    // vector memory operations a lane issues when it stores a tile (outstanding after the tile)
    // (the parity-dump instances keep the 16-byte stores: the 4-byte form would need more registers than they have)
    // (store8d: 32 RB 4-byte stores; store8t: 8 RB 16-byte stores, 8 with GELU; split partials: 16)
    [[maybe_unused]] constexpr int kStoresAfter = SPLIT ? 16 : (GELU ? kTileStoresGelu : (DBG ? 8 * RB : 32 * RB));

    using AccT = std::conditional_t<ZM, v16f, float[16]>;
    AccT acc[RB][2];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[i][c][k] = 0.F;
    v16i bias;
#pragma unroll
    for (int k = 0; k < 16; ++k) bias[k] = kBiasBits;
    KQ_ASM("" : "+v"(bias));  // opaque: never rematerialized next to an MFMA
    // P[1] starts as the bias and the metadata of "step -1" as zeros: the epilogue step 0 runs for the unit before its
    // first one adds exactly 0 (likewise at every item start)
    v16i P[2];
    P[0] = bias;
    P[1] = bias;
    v4i A[RB][CH], B0[CH], B1[2][CH];
    Meta<GPS> mt[2];
    // ZM: lanes 0-31 take the pair's first step's a_s * Q and z, lanes 32-63 the second step's (operand k = lane / 32)
    [[maybe_unused]] const bool lo = lane < 32;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int gg = 0; gg < GPS; ++gg) {
            mt[1].rec[i][gg] = v2i{0, 0};
            mt[1].z[i][gg] = 0.F;
            mt[0].z[i][gg] = 0.F;
            mt[1].as[i][gg] = 0.F;
            mt[1].az[i][gg] = 0.F;
            mt[0].as[i][gg] = 0.F;
            mt[0].az[i][gg] = 0.F;
        }

    // prologue: NS stages in flight; step 0's operands (but A row block 1) and metadata in registers
#pragma unroll
    for (int i = 0; i < NS; ++i) issue(static_cast<std::uint32_t>(i * Q::kStageBytes), 0, i);
    KQ_ASM("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    read_frags(A[0], a_lane);
    read_frags(B0, b_lane0);
    read_frags(B1[0], b_lane1);
    read_meta(mt[0], 0);

    // Step t (parity p) in four blocks (row block, column block) = b0 (0, 0), b1 (0, 1), b2 (1, 0), b3 (1, 1). An
    // epilogue unit is one block and group: per G = 128 block CH = 4 MFMAs, per G = 64 block 2, per G = 32 block two
    // units of one MFMA each. The epilogue of a unit runs in the VALU slots after the next unit's MFMAs (G = 128: after
    // MFMAs 2-4 of the next block). Reads (ds_read_b128) go into the gap after a block's first MFMA:
    //   b0: A row block 1 of step t;   b2: B column block 1 and metadata of step t + 1;
    //   b3: A row block 0 and B column block 0 of step t + 1
    //   between b1 and b2: lgkmcnt(0), vmcnt, barrier: stage t + 1 complete, stage t free; copies of step t + NS into
    //   stage t.
    // Stage t % NS is read from b2 of step t - 1 to b0 of step t; the mid-step barrier of step t comes after every
    // wave waited for those reads, and after every wave's copies of step t + 1 (issued at mid-step t + 1 - NS) landed.
    // st_now: byte offset of stage u % NS (u: the global step), st_next: of stage (u + 1) % NS; the copies of step
    // t + NS go into stage u % NS as well
    auto step_body = [&](int t, std::uint32_t st_now, std::uint32_t st_next, int r, auto parity, bool wide) __attribute__((always_inline)) {
        constexpr int p = decltype(parity)::value;
        Meta<GPS>& cur = mt[p];
        Meta<GPS>& prv = mt[p ^ 1];
        v4i (&Bc)[CH] = B1[p];
        v4i (&Bn)[CH] = B1[p ^ 1];
        const int g = (ks * steps + t) * GPS;  // global index of the step's first group
        const std::uint32_t dvo_prev = t > 0 ? dvo[RB - 1][1] : 0x80000000u;
        auto mid_step = [&]() __attribute__((always_inline)) {
            if constexpr (RB == 2) lgkm_wait<0>(A[1]);
            // the first NS - 1 steps after a tile's stores: those stores are younger than step t + 1's copies
            // (vmcnt counts to 63: a larger allowance waits for some of the stores too, which is only stricter)
            if (wide) KQ_ASM("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(min63((NS - 2) * Q::kCopies + kStoresAfter)) : "memory");
            else KQ_ASM("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * Q::kCopies) : "memory");
            issue(st_now, r, t + NS);
        };
        lgkm_wait<0>(A[0], B0, Bc, cur.rec, cur.z, cur.as, cur.az);  // step t's operands and metadata (read during step t - 1)
        if constexpr (RB == 1) {
            // 128-row tile, G = 128: two blocks b0 (0, 0), b1 (0, 1) per step; every operand of step t + 1 is read
            // during step t (after the mid-step barrier), so stage t is free at the barrier of step t as well
            // ---- b0
            mfma_first(P[0], A[0][0], B0[0], bias);
            mfma_acc(P[0], A[0][1], B0[1]);
            epi_range<0, 6, SF16, STAT, ZF, DBG>(acc[0][1], P[1], prv.rec[1][0], prv.z[1][0], prv.as[0][0], prv.az[0][0], dmp, dvo_prev, g - 1);
            mfma_acc(P[0], A[0][2], B0[2]);
            epi_range<6, 11, SF16, STAT, ZF, DBG>(acc[0][1], P[1], prv.rec[1][0], prv.z[1][0], prv.as[0][0], prv.az[0][0], dmp, dvo_prev, g - 1);
            mfma_acc(P[0], A[0][3], B0[3]);
            epi_range<11, 16, SF16, STAT, ZF, DBG>(acc[0][1], P[1], prv.rec[1][0], prv.z[1][0], prv.as[0][0], prv.az[0][0], dmp, dvo_prev, g - 1);
            // ---- b1
            mfma_first(P[1], A[0][0], Bc[0], bias);
            mid_step();
            read_frags(Bn, b_lane1 + st_next);
            read_meta(prv, st_next);
            read_frags(B0, b_lane0 + st_next);
            mfma_acc(P[1], A[0][1], Bc[1]);
            epi_range<0, 6, SF16, STAT, ZF, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            mfma_acc(P[1], A[0][2], Bc[2]);
            epi_range<6, 11, SF16, STAT, ZF, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            mfma_acc(P[1], A[0][3], Bc[3]);
            epi_range<11, 16, SF16, STAT, ZF, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            read_frags(A[0], a_lane + st_next);  // after the last MFMA that reads A[0] (and ten VALU)
        } else if constexpr (G == 128) {
            // ---- b0
            mfma_first(P[0], A[0][0], B0[0], bias);
            ds_read16<4096>(A[1][0], a_lane + st_now);
            ds_read16<5120>(A[1][1], a_lane + st_now);
            ds_read16<6144>(A[1][2], a_lane + st_now);
            ds_read16<7168>(A[1][3], a_lane + st_now);
            mfma_acc(P[0], A[0][1], B0[1]);
            epi_range<0, 6, SF16, STAT, ZFE, DBG>(acc[1][1], P[1], prv.rec[1][0], prv.z[1][0], prv.as[1][0], prv.az[1][0], dmp, dvo_prev, g - 1);
            mfma_acc(P[0], A[0][2], B0[2]);
            epi_range<6, 11, SF16, STAT, ZFE, DBG>(acc[1][1], P[1], prv.rec[1][0], prv.z[1][0], prv.as[1][0], prv.az[1][0], dmp, dvo_prev, g - 1);
            mfma_acc(P[0], A[0][3], B0[3]);
            epi_range<11, 16, SF16, STAT, ZFE, DBG>(acc[1][1], P[1], prv.rec[1][0], prv.z[1][0], prv.as[1][0], prv.az[1][0], dmp, dvo_prev, g - 1);
            // ZM, odd step t: the zero terms of the pair (t - 1, t) while both steps' metadata are in registers (prv: t - 1,
            // cur: t; prv is read again after the mid-step barrier); each MFMA follows the epilogue that last wrote its
            // block, and the next epilogue of that block comes at least a mid-step barrier later
            if constexpr (ZM) {
                if constexpr (p == 1) mfma_zero(acc[1][1], lo ? prv.az[1][0] : cur.az[1][0], lo ? prv.z[1][0] : cur.z[1][0]);
            }
            // ---- b1
            mfma_first(P[1], A[0][0], Bc[0], bias);
            mfma_acc(P[1], A[0][1], Bc[1]);
            epi_range<0, 6, SF16, STAT, ZFE, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            mfma_acc(P[1], A[0][2], Bc[2]);
            epi_range<6, 11, SF16, STAT, ZFE, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            mfma_acc(P[1], A[0][3], Bc[3]);
            epi_range<11, 16, SF16, STAT, ZFE, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            if constexpr (ZM) {
                if constexpr (p == 1) {
                    mfma_zero(acc[0][0], lo ? prv.az[0][0] : cur.az[0][0], lo ? prv.z[0][0] : cur.z[0][0]);
                    mfma_zero(acc[0][1], lo ? prv.az[0][0] : cur.az[0][0], lo ? prv.z[1][0] : cur.z[1][0]);
                    mfma_zero(acc[1][0], lo ? prv.az[1][0] : cur.az[1][0], lo ? prv.z[0][0] : cur.z[0][0]);
                }
            }
            mid_step();
            // ---- b2
            mfma_first(P[0], A[1][0], B0[0], bias);
            read_frags(Bn, b_lane1 + st_next);
            read_meta(prv, st_next);
            read_frags(A[0], a_lane + st_next);  // A row block 0 is free since b1
            mfma_acc(P[0], A[1][1], B0[1]);
            epi_range<0, 6, SF16, STAT, ZFE, DBG>(acc[0][1], P[1], cur.rec[1][0], cur.z[1][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][1], g);
            mfma_acc(P[0], A[1][2], B0[2]);
            epi_range<6, 11, SF16, STAT, ZFE, DBG>(acc[0][1], P[1], cur.rec[1][0], cur.z[1][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][1], g);
            mfma_acc(P[0], A[1][3], B0[3]);
            epi_range<11, 16, SF16, STAT, ZFE, DBG>(acc[0][1], P[1], cur.rec[1][0], cur.z[1][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][1], g);
            // ---- b3
            mfma_first(P[1], A[1][0], Bc[0], bias);
            read_frags(B0, b_lane0 + st_next);
            mfma_acc(P[1], A[1][1], Bc[1]);
            epi_range<0, 6, SF16, STAT, ZFE, DBG>(acc[1][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[1][0], cur.az[1][0], dmp, dvo[1][0], g);
            mfma_acc(P[1], A[1][2], Bc[2]);
            epi_range<6, 11, SF16, STAT, ZFE, DBG>(acc[1][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[1][0], cur.az[1][0], dmp, dvo[1][0], g);
            mfma_acc(P[1], A[1][3], Bc[3]);
            epi_range<11, 16, SF16, STAT, ZFE, DBG>(acc[1][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[1][0], cur.az[1][0], dmp, dvo[1][0], g);
        } else if constexpr (G == 64) {
            // ---- b0
            mfma_first(P[0], A[0][0], B0[0], bias);
            ds_read16<2048>(A[1][0], a_lane + st_now);
            ds_read16<3072>(A[1][1], a_lane + st_now);
            mfma_acc(P[0], A[0][1], B0[1]);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[1][1], P[1], prv.rec[1][0], prv.z[1][0], prv.as[1][0], prv.az[1][0], dmp, dvo_prev, g - 1);
            // ---- b1
            mfma_first(P[1], A[0][0], Bc[0], bias);
            mfma_acc(P[1], A[0][1], Bc[1]);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            mid_step();
            // ---- b2
            mfma_first(P[0], A[1][0], B0[0], bias);
            read_frags(Bn, b_lane1 + st_next);
            read_meta(prv, st_next);
            mfma_acc(P[0], A[1][1], B0[1]);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[0][1], P[1], cur.rec[1][0], cur.z[1][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][1], g);
            // ---- b3
            mfma_first(P[1], A[1][0], Bc[0], bias);
            read_frags(A[0], a_lane + st_next);
            read_frags(B0, b_lane0 + st_next);
            mfma_acc(P[1], A[1][1], Bc[1]);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[1][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[1][0], cur.az[1][0], dmp, dvo[1][0], g);
        } else {
            // G = 32: unit (block, k) is one MFMA over chunk k = group g + k; P[k] holds it
            // ---- b0
            mfma_first(P[0], A[0][0], B0[0], bias);
            ds_read16<2048>(A[1][0], a_lane + st_now);
            ds_read16<3072>(A[1][1], a_lane + st_now);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[1][1], P[1], prv.rec[1][1], prv.z[1][1], prv.as[1][1], prv.az[1][1], dmp, dvo_prev, g - 1);
            mfma_first(P[1], A[0][1], B0[1], bias);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[0][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][0], g);
            // ---- b1
            mfma_first(P[0], A[0][0], Bc[0], bias);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[0][0], P[1], cur.rec[0][1], cur.z[0][1], cur.as[0][1], cur.az[0][1], dmp, dvo[0][0], g + 1);
            mfma_first(P[1], A[0][1], Bc[1], bias);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[0][1], P[0], cur.rec[1][0], cur.z[1][0], cur.as[0][0], cur.az[0][0], dmp, dvo[0][1], g);
            mid_step();
            // ---- b2
            mfma_first(P[0], A[1][0], B0[0], bias);
            read_frags(Bn, b_lane1 + st_next);
            read_meta(prv, st_next);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[0][1], P[1], cur.rec[1][1], cur.z[1][1], cur.as[0][1], cur.az[0][1], dmp, dvo[0][1], g + 1);
            mfma_first(P[1], A[1][1], B0[1], bias);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[1][0], P[0], cur.rec[0][0], cur.z[0][0], cur.as[1][0], cur.az[1][0], dmp, dvo[1][0], g);
            // ---- b3
            mfma_first(P[0], A[1][0], Bc[0], bias);
            read_frags(A[0], a_lane + st_next);
            read_frags(B0, b_lane0 + st_next);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[1][0], P[1], cur.rec[0][1], cur.z[0][1], cur.as[1][1], cur.az[1][1], dmp, dvo[1][0], g + 1);
            mfma_first(P[1], A[1][1], Bc[1], bias);
            epi_range<0, 16, SF16, STAT, ZF, DBG>(acc[1][1], P[0], cur.rec[1][0], cur.z[1][0], cur.as[1][0], cur.az[1][0], dmp, dvo[1][1], g);
        }
    };
    // byte offset of stage u % NS for the global step u, advanced step by step
    constexpr std::uint32_t kRing = static_cast<std::uint32_t>(NS * Q::kStageBytes);
    auto next_stage = [](std::uint32_t st) __attribute__((always_inline)) {
        const std::uint32_t n = st + static_cast<std::uint32_t>(Q::kStageBytes);
        return n == kRing ? 0u : n;
    };
    std::uint32_t st0 = 0;
    for (int r = 0; r < items; ++r) {
        begin_item(r);
        for (int t = 0; t < steps; t += 2) {
            const std::uint32_t st1 = next_stage(st0), st2 = next_stage(st1);
            step_body(t, st0, st1, r, std::integral_constant<int, 0>{}, r > 0 && t <= NS - 2);
            step_body(t + 1, st1, st2, r, std::integral_constant<int, 1>{}, r > 0 && t + 1 <= NS - 2);
            st0 = st2;
        }
        // the reads issued in the last step (the next item's step 0 operands and metadata) land before the registers
        // they target can be given to anything else (after the last item nothing reads them)
        lgkm_wait<0>(A[0], B0, B1, mt[0].rec, mt[0].z, mt[0].as, mt[0].az);
        // drain: the epilogue of the item's last unit (block b3 and the step's last group, step steps - 1, parity 1)
        KQ_ASM("s_nop 11");
        epi_range<0, 16, SF16, STAT, ZFE, DBG>(acc[RB - 1][1], P[1], mt[1].rec[1][GPS - 1], mt[1].z[1][GPS - 1],
                                               mt[1].as[RB - 1][GPS - 1], mt[1].az[RB - 1][GPS - 1], dmp, dvo[RB - 1][1],
                                               (ks * steps + steps) * GPS - 1);

        if constexpr (SPLIT) {
            // partial tile [16 chunks][512 threads][4 floats]: chunk j of every thread is one coalesced 8 KiB run
            v4f* dst = reinterpret_cast<v4f*>(a.partial) + (static_cast<std::int64_t>(ks) * tiles + tile) * 16 * kThreads + tid;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4)
                        dst[((i * 2 + c) * 4 + q4) * kThreads] =
                            v4f{acc[i][c][4 * q4], acc[i][c][4 * q4 + 1], acc[i][c][4 * q4 + 2], acc[i][c][4 * q4 + 3]};
        } else {
            if constexpr (GELU || DBG) store8t<STAT, GELU, RB>(a, acc, m0, wm, gc, lane);
            else store8d<STAT, RB>(a, acc, m0, wm, gc, lane);
        }
        // the next item starts from zero accumulators, the bias and "step -1" metadata zeros (its step 0 operands and
        // metadata were read during this item's last step)
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int k = 0; k < 16; ++k) acc[i][c][k] = 0.F;
        P[1] = bias;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int gg = 0; gg < GPS; ++gg) {
                mt[1].rec[i][gg] = v2i{0, 0};
                mt[1].z[i][gg] = 0.F;
                mt[1].as[i][gg] = 0.F;
                mt[1].az[i][gg] = 0.F;
            }
    }
    KQ_ASM("s_waitcnt vmcnt(0)" ::: "memory");  // the copies past the range land before the workgroup ends
}

// Split K: the ranges' partial accumulators of one tile added in range order, then the same final stores.
template <bool STAT, bool GELU>
__global__ __launch_bounds__(kThreads) void gemm8_reduce_kernel(Gemm8Args a) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = tid >> 6, wm = wave & 3, wn = wave >> 2;
    const int tile = blockIdx.x;
    const int tiles = a.m_blocks * a.n_blocks;
    const int mb = tile % a.m_blocks, nbk = tile / a.m_blocks;
    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[i][c][k] = 0.F;
    for (int ks = 0; ks < a.ksplit; ++ks) {
        const v4f* src = reinterpret_cast<const v4f*>(a.partial) + (static_cast<std::int64_t>(ks) * tiles + tile) * 16 * kThreads + tid;
        v4f v[16];  // all of a range's chunks in flight at once
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = src[j * kThreads];
#pragma unroll
        for (int j = 0; j < 16; ++j) KQ_ASM("" : "+v"(v[j]));  // every load issued before the first add
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const v4f& w = v[(i * 2 + c) * 4 + q4];
                    acc[i][c][4 * q4] += w[0];
                    acc[i][c][4 * q4 + 1] += w[1];
                    acc[i][c][4 * q4 + 2] += w[2];
                    acc[i][c][4 * q4 + 3] += w[3];
                }
    }
    const int gc[2] = {col_block<GELU>(a, nbk, GELU ? wn : 2 * wn), col_block<GELU>(a, nbk, GELU ? wn + 2 : 2 * wn + 1)};
    if constexpr (GELU) store8t<STAT, true>(a, acc, mb * kBM, wm, gc, lane);
    else store8d<STAT>(a, acc, mb * kBM, wm, gc, lane);
}

// ------------------------------------------------------------------------------------------------------------------
// 128 x 160 tiles for g = 32 (gemm8w_kernel)
//
// A g = 32 projection is bound by its epilogue's VALU (two instructions per element and group, one group per MFMA),
// so its time follows the blocks a SIMD carries. Where 256 x 128 tiles leave CUs idle (the fused QKV at M = 2048,
// N = 2560: 160 tiles), 128 x 160 tiles cover the chip (256 tiles): 8 waves, wave w takes row block w % 4 and column
// blocks 0-2 (w < 4) or 3-4 (w >= 4), so the two waves of a SIMD carry five 32 x 32 blocks per k step against eight.
// One 64-column k step (two groups) per iteration; a 4-stage ring of 26 KiB stages filled by direct copies only,
// exactly four per wave and step: copy c = w + 8 j (j = 0..3) is activation fragment c (c < 8: row block c / 2, chunk
// c % 2), weight fragment c - 8 (c < 18: column block (c - 8) / 2), the activation scales of group c - 18 (c < 20),
// a 1 KiB run of weight records (c < 26: group (c - 20) / 3, column blocks 2 ((c - 20) % 3) and the next), or a
// dummy. Operands of step t + 1 are read during step t: the activation fragments and the last block's weight
// fragments into a second register set (by step parity), the other blocks' weight fragments as soon as their block's
// MFMAs are issued. Epilogue, stores and numerics are gemm8_kernel's (same operation order per element: y is
// bit-identical).
struct GeoW {
    static constexpr int kAOff = 0;                           // [4 row blocks][2 chunks][1 KiB]
    static constexpr int kBOff = kAOff + 8 * 1024;            // [5 column blocks][2 chunks][1 KiB]
    static constexpr int kSOff = kBOff + 10 * 1024;           // [2 groups][256 rows][4 B] (rows 0..127 used)
    static constexpr int kWOff = kSOff + 2 * 1024;            // [2 groups][6 column blocks][32][16 B] (block 5 unused)
    static constexpr int kStageBytes = kWOff + 2 * 3 * 1024;  // 26 KiB
    static constexpr int kStages = 4;
    static constexpr int kDummyOff = kStages * kStageBytes;
    static constexpr int kLds = kDummyOff + 1024;             // 105 KiB
    static constexpr int kCopies = 4;                         // direct copies per wave and step
};
// One copy slot of a wave for one item: source, byte offset at step 0 and per step, LDS offset within a stage (or,
// stage_mask 0, within the whole allocation: the dummy area).
struct SlotW {
    __amdgpu_buffer_rsrc_t res;
    std::uint32_t off0, inc, lds, stage_mask;
};
template <int NC>
struct MetaW {  // one k step's epilogue operands: weight records of the wave's NC column blocks, a_s of its rows
    v2i rec[NC][2];
    float as[2];
};

// Final values of a wave's NC blocks (row block wm, global column blocks gc[]), 4-byte stores as store8d: 16 per
// block and lane.
template <bool STAT, int NC>
__device__ __forceinline__ void store8w(const Gemm8Args& a, const float (&acc)[NC][16], int m0, int wm, const int (&gc)[NC], int lane) {
    const int n_out = a.N;
    const int rows = min(a.M - m0, 128);
    const __amdgpu_buffer_rsrc_t yres = rsrc(a.y + static_cast<std::int64_t>(m0) * n_out, static_cast<std::uint32_t>(rows) * n_out * 4);
    const std::uint32_t row_bytes = static_cast<std::uint32_t>(n_out) * 4;
    const bool cal = a.output_scale > 0.F;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int n = 32 * gc[c] + (lane & 31);
        const std::uint32_t col_off = n < n_out ? static_cast<std::uint32_t>(n) * 4 : 0x80000000u;
        const std::uint32_t base = col_off + static_cast<std::uint32_t>(32 * wm + 4 * (lane >> 5)) * row_bytes;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            float x = acc[c][k];
            if (STAT) x = x * a.input_scale;
            if (cal) x = calibrate_output(x, a.output_scale);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), yres, base + static_cast<std::uint32_t>(8 * (k >> 2) + (k & 3)) * row_bytes,
                                                  0, 0);
        }
    }
}

// The body of gemm8w_kernel for a wave of NC column blocks (NC = 3: waves 0-3, NC = 2: waves 4-7). Both bodies run
// the same barriers (one in the prologue, one per step).
template <int NC, bool SF16, bool STAT>
__device__ __forceinline__ void gemm8w_body(const Gemm8Args& a, std::uint8_t* lds, int wave, int lane) {
    using Q = GeoW;
    constexpr int NS = Q::kStages;
    constexpr int cb0 = NC == 3 ? 0 : 3;  // the wave's first column block in the tile
    const int wm = wave & 3;
    const std::uint32_t lds0 = lds_addr(lds);
    const int tiles = a.m_blocks * a.n_blocks;
    const int W = static_cast<int>(gridDim.x);
    const int bx = static_cast<int>(blockIdx.x);
    const int items = (tiles - bx + W - 1) / W;
    const int KC = a.K / 32;
    const int steps = a.K / 64;
    auto item_of = [&](int r) __attribute__((always_inline)) {
        int i = r * W + bx;
        if (tiles % 8 == 0) i = (i % 8) * (tiles / 8) + i / 8;
        Item it;
        it.ks = 0;
        it.tile = i;
        it.m0 = (i % a.m_blocks) * 128;
        it.nbk = i / a.m_blocks;
        return it;
    };
    const std::uint32_t meta_bytes = static_cast<std::uint32_t>(a.groups) * a.NB * 512;
    auto slot_of = [&](int j, const Item& it) __attribute__((always_inline)) {
        const int c = wave + 8 * j;
        SlotW s;
        s.stage_mask = 0xFFFFFFFFu;
        if (c < 8) {
            s.res = rsrc(a.q + static_cast<std::int64_t>(it.m0 / 32) * KC * 1024, 4u * static_cast<std::uint32_t>(KC) * 1024);
            s.off0 = static_cast<std::uint32_t>((c >> 1) * KC + (c & 1)) * 1024;
            s.inc = 2048;
            s.lds = Q::kAOff + c * 1024;
        } else if (c < 18) {
            const int f = c - 8, gcb = 5 * it.nbk + (f >> 1);
            const bool live = gcb < a.NB;
            s.res = rsrc(a.w + static_cast<std::int64_t>(live ? gcb : 0) * KC * 1024, live ? static_cast<std::uint32_t>(KC) * 1024 : 0u);
            s.off0 = static_cast<std::uint32_t>(f & 1) * 1024;
            s.inc = 2048;
            s.lds = Q::kBOff + f * 1024;
        } else if (c < 20 && !STAT) {
            const int gg = c - 18;
            s.res = rsrc(a.scale_t, static_cast<std::uint32_t>(a.groups) * a.M_p * 4);
            s.off0 = static_cast<std::uint32_t>(gg * a.M_p + it.m0) * 4;
            s.inc = static_cast<std::uint32_t>(2 * a.M_p) * 4;
            s.lds = Q::kSOff + gg * 1024;
        } else if (c >= 20 && c < 26) {
            const int gg = (c - 20) / 3, part = (c - 20) % 3;
            s.res = rsrc(a.wmeta, meta_bytes);
            s.off0 = static_cast<std::uint32_t>(gg * a.NB + 5 * it.nbk + 2 * part) * 512;
            s.inc = static_cast<std::uint32_t>(2 * a.NB) * 512;
            s.lds = Q::kWOff + gg * 3072 + part * 1024;
        } else {
            s.res = rsrc(a.wmeta, meta_bytes);
            s.off0 = 0;
            s.inc = 0;
            s.lds = Q::kDummyOff;
            s.stage_mask = 0;
        }
        return s;
    };
    auto copy = [&](const SlotW& s, std::uint32_t st, int t) __attribute__((always_inline)) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(s.res, (lds_void*)(lds + (st & s.stage_mask) + s.lds), 16, lane * 16,
                                                 s.off0 + static_cast<std::uint32_t>(t) * s.inc, 0, 0);
    };
    SlotW sl[4];
    {
        const Item it0 = item_of(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) sl[j] = slot_of(j, it0);
    }
    // issue(st, r, t): the copies of step t of item r into the stage at byte offset st; past the item, the next
    // item's steps; past the last item, the item's last step again (into a stage nothing reads any more)
    auto issue = [&](std::uint32_t st, int r, int t) __attribute__((always_inline)) {
        if (t < steps) {
#pragma unroll
            for (int j = 0; j < 4; ++j) copy(sl[j], st, t);
            return;
        }
        while (t >= steps) {
            t -= steps;
            ++r;
        }
        if (r >= items) {
#pragma unroll
            for (int j = 0; j < 4; ++j) copy(sl[j], st, steps - 1);
        } else {
            const Item it = item_of(r);
#pragma unroll
            for (int j = 0; j < 4; ++j) copy(slot_of(j, it), st, t);
        }
    };

    const int col = lane & 31;
    const std::uint32_t a_lane = lds0 + Q::kAOff + (wm * 2) * 1024 + lane * 16;
    const std::uint32_t b_lane = lds0 + Q::kBOff + (cb0 * 2) * 1024 + lane * 16;
    const std::uint32_t w_lane = lds0 + Q::kWOff + (cb0 * 32 + col) * 16;
    [[maybe_unused]] const std::uint32_t s_lane = lds0 + Q::kSOff + (32 * wm + bcast_row(lane)) * 4;
    auto read_meta = [&](MetaW<NC>& m, std::uint32_t stage) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            KQ_ASM("ds_read_b64 %0, %1 offset:%2" : "=v"(m.rec[c][0]) : "v"(w_lane + stage), "n"(c * 512));
            KQ_ASM("ds_read_b64 %0, %1 offset:%2" : "=v"(m.rec[c][1]) : "v"(w_lane + stage), "n"(3072 + c * 512));
        }
        if constexpr (!STAT) {
            KQ_ASM("ds_read_b32 %0, %1 offset:0" : "=v"(m.as[0]) : "v"(s_lane + stage));
            KQ_ASM("ds_read_b32 %0, %1 offset:1024" : "=v"(m.as[1]) : "v"(s_lane + stage));
        }
    };

    int gc[NC];
    int m0 = 0;
    Dump dmp{};
    constexpr int kStoresAfter = 16 * NC;

    float acc[NC][16];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[c][k] = 0.F;
    v16i bias;
#pragma unroll
    for (int k = 0; k < 16; ++k) bias[k] = kBiasBits;
    KQ_ASM("" : "+v"(bias));
    v16i P[2];
    P[0] = bias;
    P[1] = bias;
    v4i A[2][2], B[NC - 1][2], Bl[2][2];  // A and the last block's B by step parity; the other blocks' B single
    MetaW<NC> mt[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            mt[1].rec[c][i] = v2i{0, 0};
        }
        mt[0].as[i] = 0.F;
        mt[1].as[i] = 0.F;
    }

    // prologue: NS stages in flight; step 0's operands in registers
#pragma unroll
    for (int i = 0; i < NS; ++i) issue(static_cast<std::uint32_t>(i * Q::kStageBytes), 0, i);
    KQ_ASM("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    ds_read16<0>(A[0][0], a_lane);
    ds_read16<1024>(A[0][1], a_lane);
#pragma unroll
    for (int c = 0; c < NC - 1; ++c) {
        ds_read16<0>(B[c][0], b_lane + c * 2048);
        ds_read16<1024>(B[c][1], b_lane + c * 2048);
    }
    ds_read16<(NC - 1) * 2048>(Bl[0][0], b_lane);
    ds_read16<(NC - 1) * 2048 + 1024>(Bl[0][1], b_lane);
    read_meta(mt[0], 0);

    // Step t (parity p): units (block c, group g) in the order (0, 0), (0, 1), (1, 0), ...; each unit is one MFMA,
    // and the epilogue of a unit runs after the next unit's MFMA (the first unit's MFMA is followed by the epilogue of
    // the previous step's last unit). After unit 1: the mid-step wait and barrier (stage t + 1 complete in every
    // wave, stage t free), the copies of step t + NS into stage t, then the reads of step t + 1's operands.
    auto step_body = [&](int t, std::uint32_t st_now, std::uint32_t st_next, int r, auto parity, bool wide) __attribute__((always_inline)) {
        constexpr int p = decltype(parity)::value;
        MetaW<NC>& cur = mt[p];
        MetaW<NC>& prv = mt[p ^ 1];
        lgkm_wait<0>(A[p], B, Bl[p], cur.rec, cur.as);
        // ---- block 0
        mfma_first(P[0], A[p][0], B[0][0], bias);
        epi_range<0, 16, SF16, STAT, false, false>(acc[NC - 1], P[1], prv.rec[NC - 1][1], 0.F, prv.as[1], 0.F, dmp, 0u, 0);
        mfma_first(P[1], A[p][1], B[0][1], bias);
        epi_range<0, 16, SF16, STAT, false, false>(acc[0], P[0], cur.rec[0][0], 0.F, cur.as[0], 0.F, dmp, 0u, 0);
        if (wide) KQ_ASM("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(min63((NS - 2) * Q::kCopies + kStoresAfter)) : "memory");
        else KQ_ASM("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * Q::kCopies) : "memory");
        issue(st_now, r, t + NS);
        ds_read16<0>(A[p ^ 1][0], a_lane + st_next);
        ds_read16<1024>(A[p ^ 1][1], a_lane + st_next);
        ds_read16<(NC - 1) * 2048>(Bl[p ^ 1][0], b_lane + st_next);
        ds_read16<(NC - 1) * 2048 + 1024>(Bl[p ^ 1][1], b_lane + st_next);
        read_meta(prv, st_next);
        // ---- block 1 (NC = 2: the last block)
        const v4i& B10 = NC == 3 ? B[NC == 3 ? 1 : 0][0] : Bl[p][0];
        const v4i& B11 = NC == 3 ? B[NC == 3 ? 1 : 0][1] : Bl[p][1];
        mfma_first(P[0], A[p][0], B10, bias);
        ds_read16<0>(B[0][0], b_lane + st_next);  // block 0's operands are free: its MFMAs were issued before the barrier
        ds_read16<1024>(B[0][1], b_lane + st_next);
        epi_range<0, 16, SF16, STAT, false, false>(acc[0], P[1], cur.rec[0][1], 0.F, cur.as[1], 0.F, dmp, 0u, 0);
        mfma_first(P[1], A[p][1], B11, bias);
        epi_range<0, 16, SF16, STAT, false, false>(acc[1], P[0], cur.rec[1][0], 0.F, cur.as[0], 0.F, dmp, 0u, 0);
        if constexpr (NC == 3) {
            // ---- block 2 (the last block)
            mfma_first(P[0], A[p][0], Bl[p][0], bias);
            ds_read16<2048>(B[NC == 3 ? 1 : 0][0], b_lane + st_next);  // block 1's MFMAs were issued 32 VALU ago
            ds_read16<3072>(B[NC == 3 ? 1 : 0][1], b_lane + st_next);
            epi_range<0, 16, SF16, STAT, false, false>(acc[1], P[1], cur.rec[1][1], 0.F, cur.as[1], 0.F, dmp, 0u, 0);
            mfma_first(P[1], A[p][1], Bl[p][1], bias);
            epi_range<0, 16, SF16, STAT, false, false>(acc[2 < NC ? 2 : 0], P[0], cur.rec[2 < NC ? 2 : 0][0], 0.F, cur.as[0], 0.F, dmp, 0u, 0);
        }
    };

    constexpr std::uint32_t kRing = static_cast<std::uint32_t>(NS * Q::kStageBytes);
    auto next_stage = [](std::uint32_t st) __attribute__((always_inline)) {
        const std::uint32_t n = st + static_cast<std::uint32_t>(Q::kStageBytes);
        return n == kRing ? 0u : n;
    };
    std::uint32_t st0 = 0;
    for (int r = 0; r < items; ++r) {
        const Item it = item_of(r);
        if (r > 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) sl[j] = slot_of(j, it);
        }
        m0 = it.m0;
#pragma unroll
        for (int c = 0; c < NC; ++c) gc[c] = 5 * it.nbk + cb0 + c;
        for (int t = 0; t < steps; t += 2) {
            const std::uint32_t st1 = next_stage(st0), st2 = next_stage(st1);
            step_body(t, st0, st1, r, std::integral_constant<int, 0>{}, r > 0 && t <= NS - 2);
            step_body(t + 1, st1, st2, r, std::integral_constant<int, 1>{}, r > 0 && t + 1 <= NS - 2);
            st0 = st2;
        }
        // the reads issued in the last step (the next item's step 0 operands) land before their registers are reused
        lgkm_wait<0>(A, B, Bl, mt[0].rec, mt[0].as);
        // drain: the epilogue of the item's last unit (last block, group 1 of step steps - 1, parity 1)
        KQ_ASM("s_nop 11");
        epi_range<0, 16, SF16, STAT, false, false>(acc[NC - 1], P[1], mt[1].rec[NC - 1][1], 0.F, mt[1].as[1], 0.F, dmp, 0u, 0);
        store8w<STAT, NC>(a, acc, m0, wm, gc, lane);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[c][k] = 0.F;
        P[1] = bias;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int c = 0; c < NC; ++c) mt[1].rec[c][i] = v2i{0, 0};
            mt[1].as[i] = 0.F;
        }
    }
    KQ_ASM("s_waitcnt vmcnt(0)" ::: "memory");  // the copies past the range land before the workgroup ends
}

template <bool SF16, bool STAT>
__global__ __launch_bounds__(kThreads) void gemm8w_kernel(Gemm8Args a) {
    extern __shared__ __attribute__((aligned(16))) std::uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    if (wave < 4) gemm8w_body<3, SF16, STAT>(a, lds, wave, lane);
    else gemm8w_body<2, SF16, STAT>(a, lds, wave, lane);
}

// Measurement: the sustained int8 MFMA rate of the whole chip. Every wave of a fully resident grid (one 8-wave
// workgroup per CU, two waves per SIMD, as gemm8_kernel) issues `iters` rounds of eight independent
// v_mfma_i32_32x32x32_i8 chains (each chain's next MFMA is eight MFMAs later, so no round waits on a result) and
// nothing else; lane 0 of each wave stores its s_memtime count over the loop and the accumulators' sum, so nothing is
// dead code.
__global__ __launch_bounds__(kThreads) void mfma_ceiling_kernel(int iters, long long* cycles, int* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const v4i A = v4i{lane, lane + 1, lane + 2, lane + 3}, B = v4i{3 * lane, 1, 2, lane};
    v16i C[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int k = 0; k < 16; ++k) C[j][k] = j + k;
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) mfma_acc(C[j], A, B);
    }
    KQ_ASM("s_nop 15\n\ts_nop 15" ::: "memory");  // the last results written before they are read
    const long long t1 = __builtin_amdgcn_s_memtime();
    int r = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int k = 0; k < 16; ++k) r += C[j][k];
    if (lane == 0) {
        cycles[blockIdx.x * kWaves + wave] = t1 - t0;
        sink[blockIdx.x * kWaves + wave] = r;
    }
}

}  // namespace

// ------------------------------------------------------------------------------------------------------------------
// Host side

namespace {
// Compute units of the current device (one persistent workgroup each), cached per device.
int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}
}  // namespace

bool gemm8_eligible(const Weight& w) {
    const int g = w.geo.group;
    // k steps of 128 (g = 128) or 64 columns, walked in pairs
    return w.tiled && w.geo.bits == 4 && (g == 32 || g == 64 || g == 128) && w.geo.cols % (g == 128 ? 256 : 128) == 0 &&
           w.geo.cols_p == w.geo.cols;
}

Gemm8Plan gemm8_plan(const Weight& w, std::int64_t M, bool gelu) {
    Gemm8Plan p;
    const int NB = static_cast<int>((w.geo.rows + 31) / 32);
    p.m_blocks = static_cast<int>((M + kBM - 1) / kBM);
    p.n_blocks = gelu ? (NB / 2 + 1) / 2 : (NB + 3) / 4;
    const int k_steps = static_cast<int>(w.geo.cols / (w.geo.group == 128 ? 128 : 64));
    const int tiles = p.m_blocks * p.n_blocks;
    p.ksplit = 1;
    // g = 32 (bound by its epilogue's VALU): 128 x 160 tiles, where a SIMD carries five 32 x 32 blocks per k step
    // instead of eight (a tile costs ~0.8 of a 256 x 128 one, measured), when they fill the CUs better: where 256 x 128
    // tiles leave CUs idle and the wide tiles fill 192-256 of them (the fused QKV at M = 2048: 160 -> 256 tiles), or,
    // with 256 x 128 tiles in several rounds over the CUs, when 0.8 x the wide tiles' rounds is less (M = 4096: 2
    // rounds of 320 tiles, the second one a quarter full, against 2 full rounds of 512). Additive float zeros excluded.
    if (w.geo.group == 32 && !gelu && w.zero_mode != ZERO_FLOAT) {
        const int mw = static_cast<int>((M + 127) / 128), nw = (NB + 4) / 5, tw = mw * nw;
        const bool fill = tiles < 256 && tw >= 192 && tw <= 256 && tw > tiles;
        const bool rounds = tiles >= 256 && 4 * ((tw + 255) / 256) < 5 * ((tiles + 255) / 256);
        if (fill || rounds) {
            p.wide = true;
            p.m_blocks = mw;
            p.n_blocks = nw;
            return p;
        }
    }
    // fewer 256-row tiles than CUs: 128-row tiles fill the chip without splitting K (no partial tiles, no reduction
    // kernel), where they are enough to
    const int m128 = static_cast<int>((M + 127) / 128);
    if (w.geo.group == 128 && !gelu && tiles < 256 && m128 * p.n_blocks >= 32) {
        p.rb = 1;
        p.m_blocks = m128;
        return p;
    }
    // split K only as far as the items still fit one wave of the 256 CUs: a split that leaves some CUs with two items
    // takes as long as no split and adds the partial traffic
    for (int sp = 2; sp <= 8 && tiles * sp <= 256; sp *= 2) {
        if (k_steps % (2 * sp) || k_steps / sp < 4) break;
        p.ksplit = sp;
    }
    return p;
}

bool gemm8_fits(const LinearCall& c) {
    const Weight& w = *c.w;
    if (!w.has_prefill || !gemm8_eligible(w) || c.M <= 16) return false;
    if (c.path != PATH_BLOCKWISE && c.path != PATH_SYMMETRIC) return false;
    if (c.path == PATH_SYMMETRIC && w.zero_mode != ZERO_NONE) return false;
    if (c.gelu_gate && ((w.geo.rows / 2) % 32 || w.geo.group != 128)) return false;
    if (w.geo.rows % 4) return false;  // 16-byte output stores of four columns
    if (w.geo.rows >= (std::int64_t{1} << 21)) return false;  // a tile's output offsets (256 rows) stay below 2^31
    if ((reinterpret_cast<std::uintptr_t>(c.x) & 15u) || (c.norm_inv && (reinterpret_cast<std::uintptr_t>(c.norm_w1) & 15u)))
        return false;
    const std::int64_t M_p = round_up(c.M, kBM);
    const std::int64_t NB = (w.geo.rows + 31) / 32, groups = w.geo.cols / w.geo.group;
    if (M_p * w.geo.cols >= (std::int64_t{1} << 31) || groups * NB * 512 >= (std::int64_t{1} << 31) ||
        groups * M_p * 4 >= (std::int64_t{1} << 31) || M_p >= (std::int64_t{1} << 24))
        return false;
    return true;
}

std::size_t gemm8_partial_bytes(const Weight& w, std::int64_t M, bool gelu) {
    const Gemm8Plan p = gemm8_plan(w, M, gelu);
    if (p.ksplit == 1) return 0;
    return static_cast<std::size_t>(p.ksplit) * p.m_blocks * p.n_blocks * kThreads * 64 * 4;
}

namespace {
template <int G, int RB, bool SF16, bool STAT, bool ZF, bool GELU, bool SPLIT, bool DBG>
hipError_t launch8(const Gemm8Args& g, unsigned blocks, hipStream_t stream) {
    auto kern = gemm8_kernel<G, RB, SF16, STAT, ZF, GELU, SPLIT, DBG>;
    constexpr int lds = Geo8<G, RB>::kLds;
    static bool configured = false;  // per instance: the dynamic LDS limit is raised once
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, stream, g);
    return hipGetLastError();
}
template <bool SF16, bool STAT>
hipError_t launch8w(const Gemm8Args& g, unsigned blocks, hipStream_t stream) {
    auto kern = gemm8w_kernel<SF16, STAT>;
    static bool configured = false;  // per instance: the dynamic LDS limit is raised once
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, GeoW::kLds);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), GeoW::kLds, stream, g);
    return hipGetLastError();
}
template <int G, bool SF16, bool STAT, bool ZF, bool GELU>
hipError_t launch8_split(const Gemm8Args& g, unsigned blocks, bool split, bool dbg, hipStream_t stream) {
    if constexpr (!GELU) {  // the parity dump covers plain projections
        if (dbg) return split ? launch8<G, 2, SF16, STAT, ZF, false, true, true>(g, blocks, stream)
                              : launch8<G, 2, SF16, STAT, ZF, false, false, true>(g, blocks, stream);
    }
    return split ? launch8<G, 2, SF16, STAT, ZF, GELU, true, false>(g, blocks, stream)
                 : launch8<G, 2, SF16, STAT, ZF, GELU, false, false>(g, blocks, stream);
}
template <int G, bool SF16, bool STAT, bool ZF>
hipError_t launch8_gelu(const Gemm8Args& g, unsigned blocks, bool gelu, bool split, bool dbg, bool rb1, hipStream_t stream) {
    if constexpr (G == 128) {  // the gate/up pairing and the 128-row tile serve g = 128 weights
        if (gelu) return launch8_split<G, SF16, STAT, ZF, true>(g, blocks, split, dbg, stream);
        if (rb1) return dbg ? launch8<G, 1, SF16, STAT, ZF, false, false, true>(g, blocks, stream)
                            : launch8<G, 1, SF16, STAT, ZF, false, false, false>(g, blocks, stream);
    }
    return launch8_split<G, SF16, STAT, ZF, false>(g, blocks, split, dbg, stream);
}
template <int G>
hipError_t launch8_modes(const Gemm8Args& g, unsigned blocks, bool sf16, bool stat, bool zf, bool gelu, bool split, bool dbg,
                         bool rb1, hipStream_t stream) {
    if (sf16) {
        if (stat) return launch8_gelu<G, true, true, false>(g, blocks, gelu, split, dbg, rb1, stream);
        if (zf) return launch8_gelu<G, true, false, true>(g, blocks, gelu, split, dbg, rb1, stream);
        return launch8_gelu<G, true, false, false>(g, blocks, gelu, split, dbg, rb1, stream);
    }
    if (stat) return launch8_gelu<G, false, true, false>(g, blocks, gelu, split, dbg, rb1, stream);
    if (zf) return launch8_gelu<G, false, false, true>(g, blocks, gelu, split, dbg, rb1, stream);
    return launch8_gelu<G, false, false, false>(g, blocks, gelu, split, dbg, rb1, stream);
}
template <int G>
void launch_quantize8(const QRow8Args& q, bool stat, bool f32, bool norm, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((static_cast<std::int64_t>(q.M_p / 32) * (q.K / 128) + 3) / 4)), block(256);
#define KQ_Q8(QM, F, NM) hipLaunchKernelGGL((quantize_rows8_kernel<QM, F, NM, G>), grid, block, 0, stream, q)
    if (stat) {
        if (f32) { if (norm) KQ_Q8(QUANT_STATIC, true, true); else KQ_Q8(QUANT_STATIC, true, false); }
        else { if (norm) KQ_Q8(QUANT_STATIC, false, true); else KQ_Q8(QUANT_STATIC, false, false); }
    } else {
        if (f32) { if (norm) KQ_Q8(QUANT_DYN_SYM, true, true); else KQ_Q8(QUANT_DYN_SYM, true, false); }
        else { if (norm) KQ_Q8(QUANT_DYN_SYM, false, true); else KQ_Q8(QUANT_DYN_SYM, false, false); }
    }
#undef KQ_Q8
}
}  // namespace

hipError_t launch_gemm8(const LinearCall& c, const ActBuffers& act, hipStream_t stream, bool quantize_only, std::int8_t* d_codes,
                        float* d_scales, std::int32_t* d_sums) {
    const Weight& w = *c.w;
    const bool stat = c.path == PATH_SYMMETRIC;
    const bool zf = w.zero_mode == ZERO_FLOAT;
    const int M = static_cast<int>(c.M), K = static_cast<int>(w.geo.cols);
    const int M_p = static_cast<int>(round_up(c.M, kBM));
    const int G = w.geo.group;
    // activation quantization into the workspace
    QRow8Args q{};
    q.x = c.x;
    q.M = M;
    q.M_p = M_p;
    q.K = K;
    q.input_scale = c.input_scale;
    q.q = act.q;
    q.scale_t = act.scale;
    q.az_t = zf ? reinterpret_cast<float*>(act.sum) : nullptr;
    q.ninv = c.norm_inv;
    q.nw = c.norm_w1;
    q.d_codes = d_codes;
    q.d_scales = d_scales;
    q.d_sums = d_sums;
    {
        const bool f32 = c.x_type == ACT_F32, norm = c.norm_inv != nullptr;
        if (G == 128) launch_quantize8<128>(q, stat, f32, norm, stream);
        else if (G == 64) launch_quantize8<64>(q, stat, f32, norm, stream);
        else launch_quantize8<32>(q, stat, f32, norm, stream);
        if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    if (quantize_only) return hipSuccess;
    Gemm8Plan p = gemm8_plan(w, c.M, c.gelu_gate);
    const bool dbg = c.dump != nullptr;
    if (p.wide && dbg) {  // the parity dump runs the 256 x 128 instance (same epilogue order, so the same y)
        p.wide = false;
        p.m_blocks = static_cast<int>((c.M + kBM - 1) / kBM);
        p.n_blocks = static_cast<int>((w.geo.rows + 31) / 32 + 3) / 4;
        p.ksplit = 1;
    }
    Gemm8Args g{};
    g.q = act.q;
    g.scale_t = act.scale;
    g.az_t = reinterpret_cast<const float*>(act.sum);
    g.w = w.prefill_codes;
    g.wmeta = reinterpret_cast<const float4*>(w.prefill_meta);
    g.y = c.y;
    g.dump = c.dump;
    g.partial = act.partial;
    g.M = M;
    g.M_p = M_p;
    g.N = static_cast<int>(w.geo.rows);
    g.K = K;
    g.NB = static_cast<int>((w.geo.rows + 31) / 32);
    g.groups = K / G;
    g.m_blocks = p.m_blocks;
    g.n_blocks = p.n_blocks;
    g.ksplit = p.ksplit;
    g.input_scale = c.input_scale;
    g.output_scale = c.output_scale;
    const bool split = p.ksplit > 1, sf16 = w.scale_type == META_F16;
    const int total = p.m_blocks * p.n_blocks * p.ksplit;
    const unsigned blocks = static_cast<unsigned>(std::min(total, device_cus()));  // persistent: items loop in the kernel
    if (p.wide) {
        if (sf16) return stat ? launch8w<true, true>(g, blocks, stream) : launch8w<true, false>(g, blocks, stream);
        return stat ? launch8w<false, true>(g, blocks, stream) : launch8w<false, false>(g, blocks, stream);
    }
    hipError_t e;
    const bool rb1 = p.rb == 1;
    if (G == 128) e = launch8_modes<128>(g, blocks, sf16, stat, zf, c.gelu_gate, split, dbg, rb1, stream);
    else if (G == 64) e = launch8_modes<64>(g, blocks, sf16, stat, zf, false, split, dbg, false, stream);
    else e = launch8_modes<32>(g, blocks, sf16, stat, zf, false, split, dbg, false, stream);
    if (e != hipSuccess || !split) return e;
    const unsigned tiles = static_cast<unsigned>(p.m_blocks * p.n_blocks);
    if (stat) {
        if (c.gelu_gate) hipLaunchKernelGGL((gemm8_reduce_kernel<true, true>), dim3(tiles), dim3(kThreads), 0, stream, g);
        else hipLaunchKernelGGL((gemm8_reduce_kernel<true, false>), dim3(tiles), dim3(kThreads), 0, stream, g);
    } else {
        if (c.gelu_gate) hipLaunchKernelGGL((gemm8_reduce_kernel<false, true>), dim3(tiles), dim3(kThreads), 0, stream, g);
        else hipLaunchKernelGGL((gemm8_reduce_kernel<false, false>), dim3(tiles), dim3(kThreads), 0, stream, g);
    }
    return hipGetLastError();
}

int mfma_ceiling_workgroups() { return device_cus(); }

hipError_t launch_mfma_ceiling(int iters, long long* cycles, int* sink, hipStream_t stream) {
    hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(static_cast<unsigned>(device_cus())), dim3(kThreads), 0, stream, iters, cycles, sink);
    return hipGetLastError();
}

}  // namespace kq
