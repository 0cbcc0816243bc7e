// Skinny projection (decode, M <= 16) of the MI355X quantized linear layer: one launch per call, with the
// activation quantization fused in.
//
// Grid: one workgroup per R row tiles of 16 output rows (R = 2 with GELU gating: a gate tile and the matching up
// tile, Kidi's gate_up_proj row order, model/gemma4.cpp:308-316). The W waves of a workgroup split the K range
// into whole groups. Per chunk of its range a wave
//   1. issues the loads of the chunk's raw activations, the group metadata of its row tiles and the first T packed
//      weight tiles per row tile (16-byte loads; the activations first, so waiting for them does not wait for the
//      weights),
//   2. quantizes the chunk's activations of all M rows into its LDS region (codes in the tile's permuted order,
//      plus per-(row, group) scale, code sum and zero point) with the arithmetic of kq_device.hpp,
//   3. runs one v_mfma_i32_16x16x64_i8 (v_mfma_i32_16x16x32_i8 for g = 32) per 64-column block and row tile:
//      A = activation codes (lane = row m + 16 * k-quarter), B = the lane's own unpacked weight slot (lane =
//      output row n + 16 * k-quarter). The MFMA reduces K inside the instruction, so every finished group leaves
//      its exact int32 partial P[m][n] in the accumulator, where the group epilogue folds it into fp32.
// The waves' fp32 partials meet in LDS; one pass applies the calibrated-input scale, output calibration or GELU
// gating and stores y. Group size, chunk width and wave count are powers of two, so all indexing is shifts.
//
// Numerics: BlockwiseLinear / SymmetricPackedLinear closed forms (runtime/ynn/operators.cpp:1118-1169,
// :1250-1308): P' = sum q*u - zw*Q (2/4-bit, u = c + 2^(b-1), zw = zero point or 2^(b-1)), P' = sum q*c - zp_a*C
// (8-bit dynamic), t = s*P' (+ z*Q for additive float zeros), acc += a_s*t (dynamic) or t (calibrated).
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

constexpr int kPrefetchIters = 4;  // 64-lane quantization steps whose activation loads are issued up front
constexpr int kMaxWaves = 8;

// 8 activations of one piece: raw bits as loaded (bf16: 16 bytes in r0; f32: 32 bytes in r0, r1).
struct RawPiece {
    uint4 r0, r1;
};

__device__ __forceinline__ void piece_values(int x_type, const RawPiece& raw, float (&v)[8]) {
    if (x_type == ACT_BF16) {
        const std::uint32_t w[4] = {raw.r0.x, raw.r0.y, raw.r0.z, raw.r0.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    } else {
        v[0] = __uint_as_float(raw.r0.x);
        v[1] = __uint_as_float(raw.r0.y);
        v[2] = __uint_as_float(raw.r0.z);
        v[3] = __uint_as_float(raw.r0.w);
        v[4] = __uint_as_float(raw.r1.x);
        v[5] = __uint_as_float(raw.r1.y);
        v[6] = __uint_as_float(raw.r1.z);
        v[7] = __uint_as_float(raw.r1.w);
    }
}

// Both 16-byte loads are always issued (for bf16 the second repeats the first), so the piece needs no branch.
__device__ __forceinline__ RawPiece piece_raw(const LinearArgs& a, std::int64_t i) {
    const bool f32 = a.x_type != ACT_BF16;
    const char* base = static_cast<const char*>(a.x) + (f32 ? 4 * i : 2 * i);
    RawPiece p;
    p.r0 = *reinterpret_cast<const uint4*>(base);
    p.r1 = *reinterpret_cast<const uint4*>(base + (f32 ? 16 : 0));
    return p;
}

// Geometry of the quantization of one chunk: pieces of 8 columns, cpr = CT/8 pieces per LDS row.
struct Chunk {
    std::int64_t kb;  // first column
    int ncols;        // real columns of the chunk (<= CT)
    int lcpr;         // log2 pieces per row
    int lgc;          // log2 pieces per group
};

// Load of piece p (row m = p >> lcpr, column kk = 8 * (p & (cpr - 1))). The load is issued for every lane (a dead
// piece reads the first piece of the row block instead), so no wait is needed before later loads; `live` says
// whether the values count.
__device__ __forceinline__ RawPiece piece_load(const LinearArgs& a, const Chunk& ch, int M, int p, bool& live) {
    const int m = p >> ch.lcpr;
    const int kk = (p & ((1 << ch.lcpr) - 1)) << 3;
    live = m < M && kk < ch.ncols && ch.kb + kk < a.K;
    const std::int64_t i = live ? static_cast<std::int64_t>(m) * a.K + ch.kb + kk : 0;
    return piece_raw(a, i);
}

// Reductions over an aligned block of 2^lg lanes (lg <= 6), result in every lane of the block. Within a row of 16
// lanes the partners come from DPP (quad_perm xor 1 and xor 2, then half-row and row mirrors, which exchange
// already-uniform halves), across rows from ds_swizzle (xor 16 inside 32 lanes) and a bpermute for xor 32.
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ int swz16(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }

template <typename Op>
__device__ __forceinline__ int block_reduce(int v, int lg, Op op) {
    if (lg >= 1) v = op(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
    if (lg >= 2) v = op(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
    if (lg >= 3) v = op(v, dpp<0x141>(v));  // row_half_mirror
    if (lg >= 4) v = op(v, dpp<0x140>(v));  // row_mirror
    if (lg >= 5) v = op(v, swz16(v));
    if (lg >= 6) v = op(v, __shfl_xor(v, 32));
    return v;
}
__device__ __forceinline__ float block_max(float v, int lg) {
    return __int_as_float(block_reduce(__float_as_int(v), lg, [](int a, int b) { return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b))); }));
}
__device__ __forceinline__ float block_min(float v, int lg) {
    return __int_as_float(block_reduce(__float_as_int(v), lg, [](int a, int b) { return __float_as_int(fminf(__int_as_float(a), __int_as_float(b))); }));
}
__device__ __forceinline__ int block_sum(int v, int lg) {
    return block_reduce(v, lg, [](int a, int b) { return a + b; });
}

// Quantize piece p held by this lane; lane blocks of 2^lgc lanes (<= 64) make one (row, group) block.
template <int QM, bool DBG>
__device__ __forceinline__ void piece_quantize(const LinearArgs& a, const Chunk& ch, int M, int p, const RawPiece& raw,
                                               bool live, std::int8_t* codes, float* st_s, int* st_q, int* st_z,
                                               int lct, int lgcn, int lane, bool dump_block) {
    const int m = p >> ch.lcpr;
    const int kk = (p & ((1 << ch.lcpr) - 1)) << 3;
    const bool valid = m < M && kk < ch.ncols;
    float v[8];
    piece_values(a.x_type, raw, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = live ? v[i] : 0.F;
    float mx = 0.F, mn = 0.F;
    if (QM != QUANT_STATIC) {
#pragma unroll
        for (int i = 0; i < 8; ++i) quant_stat(QM, v[i], mx, mn);  // zeros of dead pieces change nothing
        mx = block_max(mx, ch.lgc);
        if (QM == QUANT_DYN_ASYM) mn = block_min(mn, ch.lgc);
    }
    const int bl = kk >> a.lg_group;
    const bool live_block = valid && ch.kb + kk < a.K;  // a group lies wholly inside or outside K
    const QuantBlock q = quant_block(QM, mx, mn, a.input_scale, live_block);
    std::uint32_t lo = 0, hi = 0;
    int total = 0;
    if (live) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = quant_code(QM, v[i], q, a.input_scale);
            total += c;
            if (i < 4) lo |= (static_cast<std::uint32_t>(c) & 0xFFu) << (8 * i);
            else hi |= (static_cast<std::uint32_t>(c) & 0xFFu) << (8 * (i - 4));
        }
    }
    if (valid) *reinterpret_cast<uint2*>(codes + (m << lct) + act_position(kk)) = make_uint2(lo, hi);
    total = block_sum(total, ch.lgc);
    const bool leader = (lane & ((1 << ch.lgc) - 1)) == 0;
    if (valid && leader) {
        const int sl = (m << lgcn) + bl;
        st_s[sl] = q.s;
        st_q[sl] = total;
        st_z[sl] = q.zp;
    }
    if (DBG && dump_block && live) {
        const std::int64_t k = ch.kb + kk;
        if (a.dq_codes) *reinterpret_cast<uint2*>(a.dq_codes + m * a.K + k) = make_uint2(lo, hi);
        if (leader) {
            const std::int64_t o = m * a.groups + (k >> a.lg_group);
            if (a.dq_scales) a.dq_scales[o] = q.s;
            if (a.dq_sums) a.dq_sums[o] = total;
            if (a.dq_zeros) a.dq_zeros[o] = q.zp;
        }
    }
}

// Large groups (more than 512 columns): the whole wave handles one (row, group) block at a time.
template <int QM, bool DBG>
__device__ void quantize_large(const LinearArgs& a, const Chunk& ch, int M, std::int8_t* codes, float* st_s, int* st_q,
                               int* st_z, int lct, int lgcn, int lane, bool dump_block) {
    const int gp = a.group >> 3;  // pieces per group
    for (int m = 0; m < M; ++m) {
        for (int bl = 0; bl < (ch.ncols >> a.lg_group); ++bl) {
            const std::int64_t k0 = ch.kb + (static_cast<std::int64_t>(bl) << a.lg_group);
            const bool live_block = k0 < a.K;
            float mx = 0.F, mn = 0.F;
            for (int c = lane; c < gp && live_block && QM != QUANT_STATIC; c += 64) {
                float v[8];
                piece_values(a.x_type, piece_raw(a, m * a.K + k0 + 8 * c), v);
#pragma unroll
                for (int i = 0; i < 8; ++i) quant_stat(QM, v[i], mx, mn);
            }
            mx = block_max(mx, 6);
            if (QM == QUANT_DYN_ASYM) mn = block_min(mn, 6);
            const QuantBlock q = quant_block(QM, mx, mn, a.input_scale, live_block);
            int total = 0;
            for (int c = lane; c < gp; c += 64) {
                std::uint32_t lo = 0, hi = 0;
                if (live_block) {
                    float v[8];
                    piece_values(a.x_type, piece_raw(a, m * a.K + k0 + 8 * c), v);
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int code = quant_code(QM, v[i], q, a.input_scale);
                        total += code;
                        if (i < 4) lo |= (static_cast<std::uint32_t>(code) & 0xFFu) << (8 * i);
                        else hi |= (static_cast<std::uint32_t>(code) & 0xFFu) << (8 * (i - 4));
                    }
                }
                const int kk = (bl << a.lg_group) + 8 * c;
                *reinterpret_cast<uint2*>(codes + (m << lct) + act_position(kk)) = make_uint2(lo, hi);
                if (DBG && dump_block && a.dq_codes && live_block) *reinterpret_cast<uint2*>(a.dq_codes + m * a.K + k0 + 8 * c) = make_uint2(lo, hi);
            }
            total = block_sum(total, 6);
            if (lane == 0) {
                const int sl = (m << lgcn) + bl;
                st_s[sl] = q.s;
                st_q[sl] = total;
                st_z[sl] = q.zp;
                if (DBG && dump_block && live_block) {
                    const std::int64_t o = m * a.groups + (k0 >> a.lg_group);
                    if (a.dq_scales) a.dq_scales[o] = q.s;
                    if (a.dq_sums) a.dq_sums[o] = total;
                    if (a.dq_zeros) a.dq_zeros[o] = q.zp;
                }
            }
        }
    }
}

// Group metadata entry e = (r * GC + gi) * 16 + nn of one chunk: weight scale and a second word (zero point,
// additive float zero bits or 8-bit code sum). meta_issue loads raw bits from an always-valid address (entry 0 of
// the row tile when e is outside the chunk); meta_value converts them once the weight loads are in flight.
struct MetaRaw {
    std::uint32_t s, x;
    bool ok;
};

template <int BITS, int R, int ZM, int QM>
__device__ __forceinline__ MetaRaw meta_issue(const LinearArgs& a, const std::int64_t (&nts)[R], int gb0, int ng, int lgcn,
                                              int e) {
    const int r = e >> (lgcn + 4), gi = (e >> 4) & ((1 << lgcn) - 1), nn = e & 15;
    const int rr = r < R ? r : 0;
    MetaRaw m;
    m.ok = r < R && gi < ng && nts[rr] < a.n_tiles;
    const std::int64_t mi = m.ok ? (nts[rr] * a.groups_p + gb0 + gi) * kTileRows + nn : 0;
    m.s = a.scale_half ? static_cast<std::uint32_t>(static_cast<const std::uint16_t*>(a.scales)[mi])
                       : static_cast<const std::uint32_t*>(a.scales)[mi];
    m.x = 0;
    if constexpr (BITS == 8 && QM == QUANT_DYN_ASYM) m.x = static_cast<std::uint32_t>(a.code_sums[mi]);
    if constexpr (BITS != 8 && ZM == ZERO_POINT) m.x = a.zero_points[(mi - nn) / 2 + nn / 2];
    if constexpr (BITS != 8 && ZM == ZERO_FLOAT)
        m.x = a.zero_half ? static_cast<std::uint32_t>(static_cast<const std::uint16_t*>(a.zeros)[mi])
                          : static_cast<const std::uint32_t*>(a.zeros)[mi];
    return m;
}

template <int BITS, int ZM, int QM>
__device__ __forceinline__ void meta_value(const LinearArgs& a, const MetaRaw& m, int nn, float& s, int& x2) {
    s = 0.F;
    x2 = 0;
    if (!m.ok) return;
    s = a.scale_half ? __half2float(__ushort_as_half(static_cast<unsigned short>(m.s))) : __uint_as_float(m.s);
    if constexpr (BITS == 8 && QM == QUANT_DYN_ASYM) x2 = static_cast<int>(m.x);
    if constexpr (BITS != 8 && ZM == ZERO_POINT) x2 = static_cast<int>((m.x >> (4 * (nn & 1))) & 15u);
    if constexpr (BITS != 8 && ZM == ZERO_FLOAT)
        x2 = __float_as_int(a.zero_half ? __half2float(__ushort_as_half(static_cast<unsigned short>(m.x))) : __uint_as_float(m.x));
}

// fp32 contribution of one exact partial P of group (chunk-local) gi, output row n, activation row m.
template <int BITS, int ZM, int QM, bool DBG>
__device__ __forceinline__ float group_term(const LinearArgs& a, int P, float s, int x2, const float* st_s,
                                            const int* st_q, const int* st_z, int sl, std::int64_t m, std::int64_t n,
                                            int b, bool dump_ok) {
    int Pp;
    if constexpr (BITS == 8) {
        Pp = QM == QUANT_STATIC ? P : P - st_z[sl] * x2;
    } else {
        const int zw = ZM == ZERO_POINT ? x2 : sign_offset(BITS);
        Pp = P - zw * st_q[sl];
    }
    if (DBG && a.dump && dump_ok) a.dump[(m * a.N + n) * a.groups + b] = Pp;
    float t = s * static_cast<float>(Pp);
    if constexpr (BITS != 8 && ZM == ZERO_FLOAT) t = t + __int_as_float(x2) * static_cast<float>(st_q[sl]);
    return QM == QUANT_STATIC ? t : st_s[sl] * t;
}

// QUAD (M <= 4): A row nn holds activation row m = nn & 3 restricted to the groups of slot nn >> 2 (group index
// mod 4), so one accumulator collects four groups' partials: lane (n, L), register i = partial of group slot L,
// row i. One epilogue pass then serves four groups. Otherwise A row nn is activation row nn (M <= 16) and every
// group is folded as it completes.
template <int BITS, int R, bool GELU, bool QUAD, int ZM, int QM, bool DBG>
__global__ __launch_bounds__(512) void skinny_kernel(LinearArgs a) {
    using TS = TileShape<BITS>;
    constexpr int KT = TS::KT, J = TS::J;
    constexpr int T = 4;                                   // weight tiles in flight per row tile
    constexpr int MI = (R * T * KT / 32 * 16 + 63) / 64;  // metadata entries per lane per chunk (g >= 32)
    extern __shared__ __attribute__((aligned(16))) std::uint8_t lds[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nn = lane & 15, L = lane >> 4;
    const int M = static_cast<int>(a.M);
    const int W = 1 << a.lg_waves;
    const int lg = a.lg_group;

    std::int64_t nts[R];
    if constexpr (GELU) {
        nts[0] = blockIdx.x;
        nts[1] = blockIdx.x + (a.n_tiles >> 1);
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) nts[r] = static_cast<std::int64_t>(blockIdx.x) * R + r;
    }

    const int ltpu = a.lg_tiles_per_unit;
    const int units = static_cast<int>(a.k_tiles >> ltpu);
    const int t0 = ((wave * units) >> a.lg_waves) << ltpu;
    const int t1 = (((wave + 1) * units) >> a.lg_waves) << ltpu;
    const int lct = a.lg_chunk_cols;     // log2 of the codes' LDS row stride (chunk columns)
    const int lgcn = lct - lg;           // log2 groups per chunk
    const int GC = 1 << lgcn;
    const int chunk_tiles = (1 << lct) / KT;
    const bool dump_block = DBG && blockIdx.x == 0 && (a.dq_codes || a.dq_scales);
    // A-operand row of this lane
    const int am = QUAD ? (nn & 3) : nn;
    const int aslot = nn >> 2;

    std::uint8_t* wl = lds + wave * a.wave_lds;
    std::int8_t* codes = reinterpret_cast<std::int8_t*>(wl);
    float* st_s = reinterpret_cast<float*>(wl + a.off_stats);
    int* st_q = reinterpret_cast<int*>(st_s + (M << lgcn));
    int* st_z = st_q + (M << lgcn);
    float* mt_s = reinterpret_cast<float*>(wl + a.off_meta);
    int* mt_x = reinterpret_cast<int*>(mt_s + ((R * GC) << 4));

    float acc[R][4];
    v4i C[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        C[r] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][i] = 0.F;
    }

    const uint4* wbase[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
        wbase[r] = reinterpret_cast<const uint4*>(a.tiles + (nts[r] < a.n_tiles ? nts[r] : a.n_tiles - 1) * a.k_tiles * kTileBytes) + lane;

    for (int c0 = t0; c0 < t1; c0 += chunk_tiles) {
        const int c1 = min(c0 + chunk_tiles, t1);
        Chunk ch;
        ch.kb = static_cast<std::int64_t>(c0) * KT;
        ch.ncols = (c1 - c0) * KT;
        ch.lcpr = lct - 3;
        ch.lgc = lg - 3;
        const int gb0 = static_cast<int>(ch.kb >> lg);
        const int ng = ch.ncols >> lg;
        const bool small = ch.lgc <= 6;
        const int iters = small ? ((M << ch.lcpr) + 63) >> 6 : 0;

        // 1. loads: activations, metadata, first weight batch (in this order)
        RawPiece xr[kPrefetchIters];
        bool xl[kPrefetchIters];
#pragma unroll
        for (int it = 0; it < kPrefetchIters; ++it)
            if (it < iters) xr[it] = piece_load(a, ch, M, it * 64 + lane, xl[it]);  // unset otherwise: never read
        MetaRaw mraw[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) mraw[i] = meta_issue<BITS, R, ZM, QM>(a, nts, gb0, ng, lgcn, lane + 64 * i);
        uint4 wv[R][T];
#pragma unroll
        for (int u = 0; u < T; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) wv[r][u] = load_stream(wbase[r] + static_cast<std::int64_t>(min(c0 + u, c1 - 1)) * 64);

        // 2. quantize into LDS, stage metadata
        if (small) {
#pragma unroll
            for (int it = 0; it < kPrefetchIters; ++it)
                if (it < iters)
                    piece_quantize<QM, DBG>(a, ch, M, it * 64 + lane, xr[it], xl[it], codes, st_s, st_q, st_z, lct, lgcn, lane, dump_block);
            for (int it = kPrefetchIters; it < iters; ++it) {
                bool live;
                const RawPiece raw = piece_load(a, ch, M, it * 64 + lane, live);
                piece_quantize<QM, DBG>(a, ch, M, it * 64 + lane, raw, live, codes, st_s, st_q, st_z, lct, lgcn, lane, dump_block);
            }
        } else {
            quantize_large<QM, DBG>(a, ch, M, codes, st_s, st_q, st_z, lct, lgcn, lane, dump_block);
        }
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int e = lane + 64 * i;
            if (e < ((R * GC) << 4)) {
                float sv;
                int xv;
                meta_value<BITS, ZM, QM>(a, mraw[i], nn, sv, xv);
                mt_s[e] = sv;
                mt_x[e] = xv;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // Epilogues. QUAD: groups (b_last & ~3) + L of the chunk, rows i < M. Otherwise: group b, rows 4L + i.
        auto flush_quad = [&](int r, int b_last) {
            const int b = (b_last & ~3) + L;
            const int gi = b - gb0;
            if (b >= gb0 && b <= b_last) {
                const int e = (r * GC + gi) * 16 + nn;
                const float s = mt_s[e];
                const int x2 = mt_x[e];
                const std::int64_t n = nts[r] * kTileRows + nn;
                const bool dump_ok = DBG && n < a.N && b < a.groups && nts[r] < a.n_tiles;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (i < M) acc[r][i] += group_term<BITS, ZM, QM, DBG>(a, C[r][i], s, x2, st_s, st_q, st_z, (i << lgcn) + gi, i, n, b, dump_ok);
            }
            C[r] = v4i{0, 0, 0, 0};
        };
        auto flush_group = [&](int r, int b) {
            const int gi = b - gb0;
            const int e = (r * GC + gi) * 16 + nn;
            const float s = mt_s[e];
            const int x2 = mt_x[e];
            const std::int64_t n = nts[r] * kTileRows + nn;
            const bool dump_ok = DBG && n < a.N && b < a.groups && nts[r] < a.n_tiles;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * L + i;
                if (m < M) acc[r][i] += group_term<BITS, ZM, QM, DBG>(a, C[r][i], s, x2, st_s, st_q, st_z, (m << lgcn) + gi, m, n, b, dump_ok);
            }
            C[r] = v4i{0, 0, 0, 0};
        };

        // 3. MFMA over the chunk's tiles
        const int b_chunk_last = gb0 + ng - 1;
        for (int tb = c0; tb < c1; tb += T) {
            if (tb != c0) {
#pragma unroll
                for (int u = 0; u < T; ++u)
#pragma unroll
                    for (int r = 0; r < R; ++r) wv[r][u] = load_stream(wbase[r] + static_cast<std::int64_t>(min(tb + u, c1 - 1)) * 64);
            }
#pragma unroll
            for (int u = 0; u < T; ++u) {
                const int t = tb + u;
                if (t >= c1) break;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int kcol = t * KT + 64 * j;  // first column of this 64-column block
                    v4i A = v4i{0, 0, 0, 0};
                    if constexpr (QUAD) {
                        if (lg == 5) {
                            const int b0 = kcol >> 5;
                            const bool h0 = (b0 & 3) == aslot, h1 = ((b0 + 1) & 3) == aslot;
                            if (am < M && (h0 || h1)) {
                                A = *reinterpret_cast<const v4i*>(codes + (am << lct) + (t - c0) * KT + 64 * j + 16 * L);
                                if (!h0) A.x = A.y = 0;
                                if (!h1) A.z = A.w = 0;
                            }
                        } else if (am < M && ((kcol >> lg) & 3) == aslot) {
                            A = *reinterpret_cast<const v4i*>(codes + (am << lct) + (t - c0) * KT + 64 * j + 16 * L);
                        }
                    } else {
                        if (am < M) A = *reinterpret_cast<const v4i*>(codes + (am << lct) + (t - c0) * KT + 64 * j + 16 * L);
                    }
                    // groups completed by this block
                    const int end = kcol + 64;
                    const bool done = (end & ((1 << lg) - 1)) == 0 || lg == 5;
                    const int b_last = (end >> lg) - 1;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        int o[4];
                        unpack_block_j<BITS>(wv[r][u], j, o);
                        if (QUAD || lg != 5) {
                            C[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, v4i{o[0], o[1], o[2], o[3]}, C[r], 0, 0, 0);
                            if constexpr (QUAD) {
                                if (done && ((b_last & 3) == 3 || b_last == b_chunk_last)) flush_quad(r, b_last);
                            } else {
                                if (done) flush_group(r, b_last);
                            }
                        } else {
#pragma unroll
                            for (int h = 0; h < 2; ++h) {
                                const long Ah = static_cast<long>((static_cast<std::uint64_t>(static_cast<std::uint32_t>(A[2 * h + 1])) << 32) |
                                                                  static_cast<std::uint32_t>(A[2 * h]));
                                const long Bh = static_cast<long>((static_cast<std::uint64_t>(static_cast<std::uint32_t>(o[2 * h + 1])) << 32) |
                                                                  static_cast<std::uint32_t>(o[2 * h]));
                                C[r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(Ah, Bh, C[r], 0, 0, 0);
                                flush_group(r, (kcol >> 5) + h);
                            }
                        }
                    }
                }
            }
        }
        // the next chunk overwrites this wave's LDS region
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // cross-wave reduction [W][R][16][16]: entry (4L + i, nn) is (slot L, row i) in QUAD form, row 4L + i otherwise
    float* red = reinterpret_cast<float*>(lds + a.red_off);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((wave * R + r) * 16 + 4 * L + i) * 16 + nn] = acc[r][i];
    __syncthreads();
    constexpr int OUTS = GELU ? 256 : R * 256;
    auto gather = [&](int r, int m, int c) {
        float v = 0.F;
        for (int w = 0; w < W; ++w) {
            if constexpr (QUAD) {
#pragma unroll
                for (int s = 0; s < 4; ++s) v = v + red[((w * R + r) * 16 + 4 * s + m) * 16 + c];
            } else {
                v = v + red[((w * R + r) * 16 + m) * 16 + c];
            }
        }
        if (QM == QUANT_STATIC) v = v * a.input_scale;
        return calibrate_output(v, a.output_scale);
    };
    for (int idx = threadIdx.x; idx < OUTS; idx += blockDim.x) {
        const int r = idx >> 8, m = (idx >> 4) & 15, c = idx & 15;
        if (m >= M) continue;
        if constexpr (GELU) {
            const float g = gather(0, m, c), up = gather(1, m, c);
            const std::int64_t half_n = a.N >> 1;
            const std::int64_t i = nts[0] * kTileRows + c;
            if (i < half_n) a.y[m * half_n + i] = gelu_tanh(g) * up;
        } else {
            const std::int64_t n = nts[r] * kTileRows + c;
            if (nts[r] < a.n_tiles && n < a.N) a.y[m * a.N + n] = gather(r, m, c);
        }
    }
}

int g_lds_limit = -1;

int lds_limit() {
    if (g_lds_limit < 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            v = 65536;
        g_lds_limit = std::min(v, 65536);
    }
    return g_lds_limit;
}

// Launch-shape override for tuning sweeps: KQ_SKINNY_WAVES (waves per workgroup, a power of two <= 8). Read once;
// unset means the heuristic.
int env_int(const char* name) {
    const char* v = std::getenv(name);
    return v ? std::atoi(v) : 0;
}
int tune_waves() {
    static const int v = env_int("KQ_SKINNY_WAVES");
    return v;
}

int align16(int v) { return (v + 15) / 16 * 16; }
bool pow2(std::int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
int log2i(std::int64_t v) {
    int l = 0;
    while ((std::int64_t{1} << (l + 1)) <= v) ++l;
    return l;
}

}  // namespace

// Plan of a skinny launch: waves, chunk size and LDS layout. Returns false when the call does not fit (M > 16, a
// layout the tiles cannot carry, a group size that is not a power of two, or LDS).
bool skinny_plan(const LinearCall& c, SkinnyPlan& p) {
    const Weight& w = *c.w;
    if (!w.tiled || c.path == PATH_PORTABLE || c.M < 1 || c.M > 16) return false;
    const int bits = w.geo.bits;
    const int KT = 512 / bits;
    const int g = w.geo.group;
    if (!pow2(g)) return false;
    if (bits == 2 && c.path != PATH_SYMMETRIC) return false;  // dynamic 2-bit is Kidi's portable path
    const int tpu = g > KT ? g / KT : 1;
    const int units = static_cast<int>(w.geo.k_tiles / tpu);
    p.R = c.gelu_gate ? 2 : 1;
    if (c.gelu_gate && (w.geo.rows / 2) % kTileRows) return false;
    p.blocks = c.gelu_gate ? w.geo.n_tiles / 2 : (w.geo.n_tiles + p.R - 1) / p.R;
    // waves: about 2048 in flight over the chip, whole units per wave, a power of two
    int W = static_cast<int>(std::max<std::int64_t>(1, 2048 / std::max<std::int64_t>(1, p.blocks)));
    W = std::min({W, kMaxWaves, units});
    if (tune_waves() > 0) W = std::min({tune_waves(), kMaxWaves, units});
    W = 1 << log2i(W);
    const int per_wave_tiles = (units + W - 1) / W * tpu;
    p.T = 4;
    int chunk = std::max(tpu, p.T);
    chunk = std::min<int>(chunk, std::max<int>(tpu, 1 << (log2i(per_wave_tiles - 1) + 1)));  // pow2 >= per-wave tiles
    if (per_wave_tiles == 1) chunk = std::max(tpu, 1);
    const int CT = chunk * KT;
    const int GC = CT / g;
    const int M = static_cast<int>(c.M);
    p.chunk_tiles = chunk;
    p.off_stats = align16(M * CT);
    p.off_meta = p.off_stats + align16(12 * M * GC);
    p.wave_lds = p.off_meta + align16(8 * p.R * GC * 16);
    const int limit = lds_limit();
    while (W > 1 && W * p.wave_lds + W * p.R * 1024 > limit) W >>= 1;
    if (W * p.wave_lds + W * p.R * 1024 > limit) return false;
    p.W = W;
    p.red_off = W * p.wave_lds;
    p.lds_bytes = p.red_off + W * p.R * 1024;
    return true;
}

hipError_t launch_skinny(const LinearCall& c, const SkinnyPlan& p, hipStream_t stream) {
    dev::LinearArgs a = dev::make_linear_args(c);
    const int KT = 512 / c.w->geo.bits;
    a.quant_mode = c.path == PATH_SYMMETRIC ? dev::QUANT_STATIC : (c.w->geo.bits == 8 ? dev::QUANT_DYN_ASYM : dev::QUANT_DYN_SYM);
    a.scale_half = c.w->scale_type == META_F16;
    a.chunk_tiles = p.chunk_tiles;
    a.wave_lds = p.wave_lds;
    a.off_stats = p.off_stats;
    a.off_meta = p.off_meta;
    a.red_off = p.red_off;
    a.lg_group = log2i(c.w->geo.group);
    a.lg_chunk_cols = log2i(static_cast<std::int64_t>(p.chunk_tiles) * KT);
    a.lg_waves = log2i(p.W);
    a.lg_tiles_per_unit = c.w->geo.group > KT ? log2i(c.w->geo.group / KT) : 0;
    const dim3 grid(static_cast<unsigned>(p.blocks)), block(64 * p.W);
    const std::size_t lds = static_cast<std::size_t>(p.lds_bytes);
    const bool quad = c.M <= 4;
    const int zm = c.w->zero_mode;
    const bool stat = c.path == PATH_SYMMETRIC;
    const bool dbg = c.dump || c.dq_codes || c.dq_scales || c.dq_sums || c.dq_zeros;
#define KQ_SK(B, Q, ZM, QM)                                                                                              \
    do {                                                                                                                 \
        if (c.gelu_gate) hipLaunchKernelGGL((skinny_kernel<B, 2, true, Q, ZM, QM, false>), grid, block, lds, stream, a); \
        else if (dbg) hipLaunchKernelGGL((skinny_kernel<B, 1, false, Q, ZM, QM, true>), grid, block, lds, stream, a);    \
        else hipLaunchKernelGGL((skinny_kernel<B, 1, false, Q, ZM, QM, false>), grid, block, lds, stream, a);            \
    } while (0)
#define KQ_SK_Q(B, ZM, QM)            \
    do {                              \
        if (quad) KQ_SK(B, true, ZM, QM); \
        else KQ_SK(B, false, ZM, QM); \
    } while (0)
    switch (c.w->geo.bits) {
    case 2:  // dynamic 2-bit is the portable path; the skinny kernel serves the calibrated form
        KQ_SK_Q(2, ZERO_NONE, dev::QUANT_STATIC);
        break;
    case 4:
        if (stat) KQ_SK_Q(4, ZERO_NONE, dev::QUANT_STATIC);
        else if (zm == ZERO_POINT) KQ_SK_Q(4, ZERO_POINT, dev::QUANT_DYN_SYM);
        else if (zm == ZERO_FLOAT) KQ_SK_Q(4, ZERO_FLOAT, dev::QUANT_DYN_SYM);
        else KQ_SK_Q(4, ZERO_NONE, dev::QUANT_DYN_SYM);
        break;
    default:
        if (stat) KQ_SK_Q(8, ZERO_NONE, dev::QUANT_STATIC);
        else KQ_SK_Q(8, ZERO_NONE, dev::QUANT_DYN_ASYM);
        break;
    }
#undef KQ_SK_Q
#undef KQ_SK
    return hipGetLastError();
}

}  // namespace kq
