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
constexpr int kMaxWaves = 16;
constexpr std::uint32_t kOob = 0x80000000u;  // buffer offset past every resource: the load returns zeros
constexpr int kRsrcWord3 = 0x00020000;       // raw (unformatted) buffer resource, gfx9-family word 3

// Buffer resource over [base, base + bytes): loads at 32-bit byte offsets, zeros outside the range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kRsrcWord3);
}
__device__ __forceinline__ uint4 buf_b128(__amdgpu_buffer_rsrc_t r, std::uint32_t off) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 8 activations of one piece: raw bits as loaded (bf16: 16 bytes in r0; f32: 32 bytes in r0, r1).
struct RawPiece {
    uint4 r0, r1;
};

__device__ __forceinline__ void piece_values(bool f32, const RawPiece& raw, float (&v)[8]) {
    if (!f32) {
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

// Geometry of the quantization of one chunk: pieces of 8 columns, cpr = CT/8 pieces per LDS row.
struct Chunk {
    std::int64_t kb;  // first column
    int ncols;        // real columns of the chunk (<= CT)
    int lcpr;         // log2 pieces per row
    int lgc;          // log2 pieces per group
};

// Piece p: row m = p >> lcpr, chunk column kk = 8 * (p & (cpr - 1)). Both 16-byte loads are always issued (the
// second repeats the first for bf16); a piece outside the rows, the chunk or K reads zeros.
__device__ __forceinline__ RawPiece piece_load(const LinearArgs& a, __amdgpu_buffer_rsrc_t xr, bool f32, const Chunk& ch,
                                               int M, int p) {
    const int m = p >> ch.lcpr;
    const int kk = (p & ((1 << ch.lcpr) - 1)) << 3;
    const bool live = m < M && kk < ch.ncols && ch.kb + kk < a.K;
    const std::uint32_t e = static_cast<std::uint32_t>(m * a.K + ch.kb + kk);
    const std::uint32_t off = live ? (f32 ? e * 4 : e * 2) : kOob;
    RawPiece r;
    r.r0 = buf_b128(xr, off);
    r.r1 = buf_b128(xr, f32 ? off + 16 : off);
    return r;
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

// Per-wave LDS region: codes [M][CT] (permuted order), stats [M][GC] x {scale, sum, zero point}, the chunk's raw
// metadata per row tile (scale block, second-word block), its weight tiles [R][chunk tiles][1 KiB] and a 16-byte
// zero slot that inactive A-operand lanes read.
struct WaveLds {
    std::int8_t* codes;
    float* st_s;
    int* st_q;
    int* st_z;
};

// Quantize the piece this lane loaded; lane blocks of 2^lgc lanes (<= 64) make one (row, group) block. Dead pieces
// hold zeros, so they add nothing to a block's statistics; they only skip the stores.
template <int QM, bool DBG>
__device__ __forceinline__ void piece_quantize(const LinearArgs& a, bool f32, const Chunk& ch, int M, int p,
                                               const RawPiece& raw, const WaveLds& w, int lct, int lgcn, int lane,
                                               bool dump_block) {
    const int m = p >> ch.lcpr;
    const int kk = (p & ((1 << ch.lcpr) - 1)) << 3;
    const bool valid = m < M && kk < ch.ncols;
    float v[8];
    piece_values(f32, raw, v);
    float mx = 0.F, mn = 0.F;
    if (QM != QUANT_STATIC) {
#pragma unroll
        for (int i = 0; i < 8; ++i) quant_stat(QM, v[i], mx, mn);
        mx = block_max(mx, ch.lgc);
        if (QM == QUANT_DYN_ASYM) mn = block_min(mn, ch.lgc);
    }
    const int bl = kk >> a.lg_group;
    const bool live_block = valid && ch.kb + kk < a.K;  // a group lies wholly inside or outside K
    const QuantBlock q = quant_block(QM, mx, mn, a.input_scale, live_block);
    std::uint32_t lo = 0, hi = 0;
    int total = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int c = quant_code(QM, v[i], q, a.input_scale);
        total += c;
        if (i < 4) lo |= (static_cast<std::uint32_t>(c) & 0xFFu) << (8 * i);
        else hi |= (static_cast<std::uint32_t>(c) & 0xFFu) << (8 * (i - 4));
    }
    if (valid) *reinterpret_cast<uint2*>(w.codes + (m << lct) + act_position(kk)) = make_uint2(lo, hi);
    total = block_sum(total, ch.lgc);
    const bool leader = (lane & ((1 << ch.lgc) - 1)) == 0;
    if (valid && leader) {
        const int sl = (m << lgcn) + bl;
        w.st_s[sl] = q.s;
        w.st_q[sl] = total;
        w.st_z[sl] = q.zp;
    }
    if (DBG && dump_block && live_block) {
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
__device__ void quantize_large(const LinearArgs& a, __amdgpu_buffer_rsrc_t xr, bool f32, const Chunk& ch, int M,
                               const WaveLds& w, int lct, int lgcn, int lane, bool dump_block) {
    const int gp = a.group >> 3;  // pieces per group
    for (int m = 0; m < M; ++m) {
        for (int bl = 0; bl < (ch.ncols >> a.lg_group); ++bl) {
            const std::int64_t k0 = ch.kb + (static_cast<std::int64_t>(bl) << a.lg_group);
            const bool live_block = k0 < a.K;
            auto load = [&](int c) {
                const std::uint32_t e = static_cast<std::uint32_t>(m * a.K + k0 + 8 * c);
                const std::uint32_t off = live_block ? (f32 ? e * 4 : e * 2) : kOob;
                RawPiece r;
                r.r0 = buf_b128(xr, off);
                r.r1 = buf_b128(xr, f32 ? off + 16 : off);
                return r;
            };
            float mx = 0.F, mn = 0.F;
            if (QM != QUANT_STATIC) {
                for (int c = lane; c < gp; c += 64) {
                    float v[8];
                    piece_values(f32, load(c), v);
#pragma unroll
                    for (int i = 0; i < 8; ++i) quant_stat(QM, v[i], mx, mn);
                }
                mx = block_max(mx, 6);
                if (QM == QUANT_DYN_ASYM) mn = block_min(mn, 6);
            }
            const QuantBlock q = quant_block(QM, mx, mn, a.input_scale, live_block);
            int total = 0;
            for (int c = lane; c < gp; c += 64) {
                float v[8];
                piece_values(f32, load(c), v);
                std::uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int code = quant_code(QM, v[i], q, a.input_scale);
                    total += code;
                    if (i < 4) lo |= (static_cast<std::uint32_t>(code) & 0xFFu) << (8 * i);
                    else hi |= (static_cast<std::uint32_t>(code) & 0xFFu) << (8 * (i - 4));
                }
                const int kk = (bl << a.lg_group) + 8 * c;
                *reinterpret_cast<uint2*>(w.codes + (m << lct) + act_position(kk)) = make_uint2(lo, hi);
                if (DBG && dump_block && a.dq_codes && live_block) *reinterpret_cast<uint2*>(a.dq_codes + m * a.K + k0 + 8 * c) = make_uint2(lo, hi);
            }
            total = block_sum(total, 6);
            if (lane == 0) {
                const int sl = (m << lgcn) + bl;
                w.st_s[sl] = q.s;
                w.st_q[sl] = total;
                w.st_z[sl] = q.zp;
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

// fp32 contribution of one exact partial P of a group, output row n, activation row m; s = weight scale, x2 = the
// group's second word (zero point, additive float zero bits or 8-bit code sum), sl = the (row, group) stats slot.
template <int BITS, int ZM, int QM, bool DBG>
__device__ __forceinline__ float group_term(const LinearArgs& a, int P, float s, int x2, const WaveLds& w, int sl,
                                            std::int64_t m, std::int64_t n, int b, bool dump_ok) {
    int Pp;
    if constexpr (BITS == 8) {
        Pp = QM == QUANT_STATIC ? P : P - w.st_z[sl] * x2;
    } else {
        const int zw = ZM == ZERO_POINT ? x2 : sign_offset(BITS);
        Pp = P - zw * w.st_q[sl];
    }
    if (DBG && dump_ok) a.dump[(m * a.N + n) * a.groups + b] = Pp;
    float t = s * static_cast<float>(Pp);
    if constexpr (BITS != 8 && ZM == ZERO_FLOAT) t = t + __int_as_float(x2) * static_cast<float>(w.st_q[sl]);
    return QM == QUANT_STATIC ? t : w.st_s[sl] * t;
}

typedef __attribute__((address_space(3))) void lds_void;

// Direct-to-LDS copy of `bytes` from a buffer resource in steps of 64 * SIZE bytes: lane l of a step writes bytes
// [step + SIZE*l, step + SIZE*(l+1)) of dst. Bytes past the resource read as zeros, so dst must hold whole steps.
template <int SIZE>
__device__ __forceinline__ void dma(__amdgpu_buffer_rsrc_t r, std::uint8_t* dst, int bytes, int lane) {
    for (int off = 0; off < bytes; off += 64 * SIZE) {
        if constexpr (SIZE == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + off), 16, off + lane * 16, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + off), 4, off + lane * 4, 0, 0, 0);
    }
}

// Raw metadata of group slot gi, row nn, from the chunk's LDS copies (scale block and second-word block of one row
// tile, in the global layouts: scales [group][16] F16|F32, zero points [group][8 bytes of nibble pairs], code sums
// [group][16] I32, float zeros [group][16] F16|F32).
template <int BITS, int ZM, int QM>
__device__ __forceinline__ void meta_at(const LinearArgs& a, const std::uint8_t* sblk, const std::uint8_t* xblk, int gi, int nn,
                                        float& s, int& x2) {
    const int e = gi * 16 + nn;
    s = a.scale_half ? __half2float(*reinterpret_cast<const __half*>(sblk + 2 * e)) : *reinterpret_cast<const float*>(sblk + 4 * e);
    x2 = 0;
    if constexpr (BITS == 8 && QM == QUANT_DYN_ASYM) x2 = *reinterpret_cast<const int*>(xblk + 4 * e);
    if constexpr (BITS != 8 && ZM == ZERO_POINT) x2 = (xblk[gi * 8 + (nn >> 1)] >> (4 * (nn & 1))) & 15;
    if constexpr (BITS != 8 && ZM == ZERO_FLOAT)
        x2 = __float_as_int(a.zero_half ? __half2float(*reinterpret_cast<const __half*>(xblk + 2 * e)) : *reinterpret_cast<const float*>(xblk + 4 * e));
}

// Weight codes of 64-column block j (runtime) of a slot, for loops that stay rolled: the block's bytes of the slot
// are (4-bit) dwords 2j, 2j+1, (2-bit) dword j, (8-bit) all four.
template <int BITS>
__device__ __forceinline__ v4i slot_block(const std::uint8_t* slot, int j) {
    int o[4];
    if constexpr (BITS == 8) {
        const v4i v = *reinterpret_cast<const v4i*>(slot);
        return v;
    } else if constexpr (BITS == 4) {
        const uint2 d = *reinterpret_cast<const uint2*>(slot + 8 * j);
        o[0] = static_cast<int>(d.x & 0x0F0F0F0Fu);
        o[1] = static_cast<int>((d.x >> 4) & 0x0F0F0F0Fu);
        o[2] = static_cast<int>(d.y & 0x0F0F0F0Fu);
        o[3] = static_cast<int>((d.y >> 4) & 0x0F0F0F0Fu);
    } else {
        const std::uint32_t d = *reinterpret_cast<const std::uint32_t*>(slot + 4 * j);
        o[0] = static_cast<int>(d & 0x03030303u);
        o[1] = static_cast<int>((d >> 2) & 0x03030303u);
        o[2] = static_cast<int>((d >> 4) & 0x03030303u);
        o[3] = static_cast<int>((d >> 6) & 0x03030303u);
    }
    return v4i{o[0], o[1], o[2], o[3]};
}

// QUAD (M <= 4): A row nn holds activation row m = nn & 3 restricted to the groups of slot nn >> 2 (group index
// mod 4), so one accumulator collects four groups' partials: lane (n, L), register i = partial of group slot L,
// row i; one epilogue pass serves four groups and always falls on a 64-column block boundary. Otherwise A row nn
// is activation row nn (M <= 16) and every group is folded as it completes.
//
// Per chunk of a wave's K range: (1) the first activation piece is loaded into registers, then the chunk's group
// metadata and weight tiles of every row tile are copied straight into the wave's LDS (buffer_load ... lds); (2)
// the activations are quantized into LDS; (3) one rolled loop walks the chunk's 64-column blocks: an A read, per
// row tile a B read + unpack + MFMA, and the epilogue when a group (quad) completes. Rolled loops keep the code the
// waves walk through short: every kernel launch starts with cold instruction caches.
template <int BITS, int R, bool GELU, bool QUAD, int ZM, int QM, bool DBG>
__global__ __launch_bounds__(1024) void skinny_kernel(LinearArgs a) {
    using TS = TileShape<BITS>;
    constexpr int KT = TS::KT, J = TS::J;
    constexpr int LJ = J == 1 ? 0 : (J == 2 ? 1 : 2);
    extern __shared__ __attribute__((aligned(16))) std::uint8_t lds[];

    // the wave index is uniform within the wave: keep it (and all range and loop arithmetic) in scalar registers
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nn = lane & 15, L = lane >> 4;
    const int M = static_cast<int>(a.M);
    const int W = 1 << a.lg_waves;
    const int lg = a.lg_group;
    const bool f32 = a.x_type != ACT_BF16;

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
    const int chunk_tiles = (1 << lct) / KT;
    const bool dump_block = DBG && blockIdx.x == 0 && (a.dq_codes || a.dq_scales);
    const int am = QUAD ? (nn & 3) : nn;  // A-operand row of this lane
    const int aslot = nn >> 2;

    std::uint8_t* wl = lds + wave * a.wave_lds;
    WaveLds w;
    w.codes = reinterpret_cast<std::int8_t*>(wl);
    w.st_s = reinterpret_cast<float*>(wl + a.off_stats);
    w.st_q = reinterpret_cast<int*>(w.st_s + (M << lgcn));
    w.st_z = w.st_q + (M << lgcn);
    const int zero_slot = a.wave_lds - 16;  // 16 zero bytes for inactive A lanes
    if (lane == 0) *reinterpret_cast<uint4*>(wl + zero_slot) = make_uint4(0, 0, 0, 0);

    const __amdgpu_buffer_rsrc_t xres = rsrc(a.x, static_cast<std::uint32_t>(a.M * a.K * (f32 ? 4 : 2)));
    const int ssz = a.scale_half ? 2 : 4;

    float acc[R][4];
    v4i C[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        C[r] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][i] = 0.F;
    }

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

        // 1. loads: the first activation piece (registers), then metadata and weight tiles (straight into LDS)
        const RawPiece first = piece_load(a, xres, f32, ch, M, lane);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const std::int64_t nt = nts[r] < a.n_tiles ? nts[r] : a.n_tiles - 1;
            const std::int64_t e0 = (nt * a.groups_p + gb0) * kTileRows;  // first metadata entry of the chunk
            const std::uint32_t live = nts[r] < a.n_tiles ? 1u : 0u;
            dma<4>(rsrc(static_cast<const std::uint8_t*>(a.scales) + e0 * ssz, live * ng * 16 * ssz), wl + a.off_meta + r * a.scale_block,
                   ng * 16 * ssz, lane);
            if constexpr (BITS == 8 && QM == QUANT_DYN_ASYM)
                dma<4>(rsrc(a.code_sums + e0, live * ng * 64), wl + a.off_x2 + r * a.x2_block, ng * 64, lane);
            if constexpr (BITS != 8 && ZM == ZERO_POINT)
                dma<4>(rsrc(a.zero_points + e0 / 2, live * ng * 8), wl + a.off_x2 + r * a.x2_block, ng * 8, lane);
            if constexpr (BITS != 8 && ZM == ZERO_FLOAT) {
                const int zsz = a.zero_half ? 2 : 4;
                dma<4>(rsrc(static_cast<const std::uint8_t*>(a.zeros) + e0 * zsz, live * ng * 16 * zsz), wl + a.off_x2 + r * a.x2_block,
                       ng * 16 * zsz, lane);
            }
            dma<16>(rsrc(a.tiles + (nt * a.k_tiles + c0) * kTileBytes, static_cast<std::uint32_t>((c1 - c0) * kTileBytes)),
                    wl + a.off_w + r * chunk_tiles * kTileBytes, (c1 - c0) * kTileBytes, lane);
        }

        // 2. quantize the chunk's activations into LDS
        if (small) {
            for (int it = 0; it < iters; ++it) {
                const int p = it * 64 + lane;
                const RawPiece raw = it == 0 ? first : piece_load(a, xres, f32, ch, M, p);
                piece_quantize<QM, DBG>(a, f32, ch, M, p, raw, w, lct, lgcn, lane, dump_block);
            }
        } else {
            quantize_large<QM, DBG>(a, xres, f32, ch, M, w, lct, lgcn, lane, dump_block);
        }
        __builtin_amdgcn_s_waitcnt(0);  // the LDS copies and the codes are complete
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // 3. one rolled loop over the chunk's 64-column blocks; the next block's A and B operands are read from LDS
        //    while this block's MFMAs run
        const int blocks = (c1 - c0) * J;
        const int b_chunk_last = gb0 + ng - 1;
        auto read_a = [&](int blk) {
            const int u = blk >> LJ, j = blk & (J - 1);
            const int kcol = (c0 + u) * KT + 64 * j;
            const int code_off = (am << lct) + u * KT + 64 * j + 16 * L;
            if (QUAD && lg == 5) {
                const int b0 = kcol >> 5;
                const int o0 = (am < M && (b0 & 3) == aslot) ? code_off : zero_slot;
                const int o1 = (am < M && ((b0 + 1) & 3) == aslot) ? code_off + 8 : zero_slot;
                const uint2 lo = *reinterpret_cast<const uint2*>(wl + o0);
                const uint2 hi = *reinterpret_cast<const uint2*>(wl + o1);
                return v4i{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(hi.x), static_cast<int>(hi.y)};
            }
            const bool on = QUAD ? (am < M && ((kcol >> lg) & 3) == aslot) : am < M;
            return *reinterpret_cast<const v4i*>(wl + (on ? code_off : zero_slot));
        };
        auto read_b = [&](int blk, int r) {
            const int u = blk >> LJ, j = blk & (J - 1);
            return slot_block<BITS>(wl + a.off_w + (r * chunk_tiles + u) * kTileBytes + 16 * lane, j);
        };
        v4i An = read_a(0), Bn[R];
#pragma unroll
        for (int r = 0; r < R; ++r) Bn[r] = read_b(0, r);
        for (int blk = 0; blk < blocks; ++blk) {
            const v4i A = An;
            v4i B[R];
#pragma unroll
            for (int r = 0; r < R; ++r) B[r] = Bn[r];
            const int nb = blk + 1 < blocks ? blk + 1 : blk;  // the last iteration re-reads its own block
            An = read_a(nb);
#pragma unroll
            for (int r = 0; r < R; ++r) Bn[r] = read_b(nb, r);
            const int u = blk >> LJ, j = blk & (J - 1);
            const int kcol = (c0 + u) * KT + 64 * j;  // first column of this 64-column block
            const int end = kcol + 64;
            const bool done = lg == 5 || (end & ((1 << lg) - 1)) == 0;
            const int b_last = (end >> lg) - 1;
            const bool flush = QUAD ? (done && ((b_last & 3) == 3 || b_last == b_chunk_last)) : done;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (QUAD || lg != 5) {
                    C[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B[r], C[r], 0, 0, 0);
                } else {
                    // M > 4 with g = 32: two groups per block, each folded after its own 32-column MFMA
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const long Ah = static_cast<long>((static_cast<std::uint64_t>(static_cast<std::uint32_t>(A[2 * h + 1])) << 32) |
                                                          static_cast<std::uint32_t>(A[2 * h]));
                        const long Bh = static_cast<long>((static_cast<std::uint64_t>(static_cast<std::uint32_t>(B[r][2 * h + 1])) << 32) |
                                                          static_cast<std::uint32_t>(B[r][2 * h]));
                        C[r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(Ah, Bh, C[r], 0, 0, 0);
                        if (h == 0) {
                            const int b = kcol >> 5, gi = b - gb0;
                            float sv;
                            int x2;
                            meta_at<BITS, ZM, QM>(a, wl + a.off_meta + r * a.scale_block, wl + a.off_x2 + r * a.x2_block, gi, nn, sv, x2);
                            const std::int64_t n = nts[r] * kTileRows + nn;
                            const bool dump_ok = DBG && a.dump && n < a.N && b < a.groups && nts[r] < a.n_tiles;
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int m = 4 * L + i;
                                if (m < M) acc[r][i] += group_term<BITS, ZM, QM, DBG>(a, C[r][i], sv, x2, w, (m << lgcn) + gi, m, n, b, dump_ok);
                            }
                            C[r] = v4i{0, 0, 0, 0};
                        }
                    }
                }
            }
            if (flush) {
                // QUAD: group (b_last & ~3) + L of the chunk, rows i < M. Otherwise: group b_last, rows 4L + i.
                const int b = QUAD ? (b_last & ~3) + L : b_last;
                const int gi = b - gb0;
                const bool on = !QUAD || (b >= gb0 && b <= b_last);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (on) {
                        float sv;
                        int x2;
                        meta_at<BITS, ZM, QM>(a, wl + a.off_meta + r * a.scale_block, wl + a.off_x2 + r * a.x2_block, gi, nn, sv, x2);
                        const std::int64_t n = nts[r] * kTileRows + nn;
                        const bool dump_ok = DBG && a.dump && n < a.N && b < a.groups && nts[r] < a.n_tiles;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int m = QUAD ? i : 4 * L + i;
                            if (m < M) acc[r][i] += group_term<BITS, ZM, QM, DBG>(a, C[r][i], sv, x2, w, (m << lgcn) + gi, m, n, b, dump_ok);
                        }
                    }
                    C[r] = v4i{0, 0, 0, 0};
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
    for (int idx = threadIdx.x; idx < OUTS; idx += blockDim.x) {
        const int r = idx >> 8, m = (idx >> 4) & 15, c = idx & 15;
        if (m >= M) continue;
        float v[2] = {0.F, 0.F};
#pragma unroll
        for (int h = 0; h < (GELU ? 2 : 1); ++h) {
            const int rr = GELU ? h : r;
            for (int wv2 = 0; wv2 < W; ++wv2) {
                if constexpr (QUAD) {
#pragma unroll
                    for (int sl = 0; sl < 4; ++sl) v[h] = v[h] + red[((wv2 * R + rr) * 16 + 4 * sl + m) * 16 + c];
                } else {
                    v[h] = v[h] + red[((wv2 * R + rr) * 16 + m) * 16 + c];
                }
            }
            if (QM == QUANT_STATIC) v[h] = v[h] * a.input_scale;
            v[h] = calibrate_output(v[h], a.output_scale);
        }
        if constexpr (GELU) {
            const std::int64_t half_n = a.N >> 1;
            const std::int64_t i = nts[0] * kTileRows + c;
            if (i < half_n) a.y[m * half_n + i] = gelu_tanh(v[0]) * v[1];
        } else {
            const std::int64_t nt = static_cast<std::int64_t>(blockIdx.x) * R + r;
            const std::int64_t n = nt * kTileRows + c;
            if (nt < a.n_tiles && n < a.N) a.y[m * a.N + n] = v[0];
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
    // buffer resources address with 32-bit offsets
    if (w.geo.k_tiles * kTileBytes >= (std::int64_t{1} << 31) || w.geo.meta_count() * 4 >= (std::int64_t{1} << 31) ||
        c.M * w.geo.cols * 4 >= (std::int64_t{1} << 31))
        return false;
    // two row tiles per workgroup when there are enough of them (halves the redundant activation quantization)
    p.R = c.gelu_gate ? 2 : 1;
    if (c.gelu_gate && (w.geo.rows / 2) % kTileRows) return false;
    p.blocks = c.gelu_gate ? w.geo.n_tiles / 2 : (w.geo.n_tiles + p.R - 1) / p.R;
    // waves: about 4096 over the chip (four per SIMD), whole units per wave, a power of two
    int W = static_cast<int>(std::max<std::int64_t>(1, 4096 / std::max<std::int64_t>(1, p.blocks)));
    W = std::min({W, kMaxWaves, units});
    W = 1 << log2i(W);
    const int per_wave_tiles = (units + W - 1) / W * tpu;
    p.T = 4;
    int chunk = std::max(tpu, p.T);
    chunk = std::min<int>(chunk, std::max<int>(tpu, 1 << (log2i(per_wave_tiles - 1) + 1)));  // pow2 >= per-wave tiles
    if (per_wave_tiles == 1) chunk = std::max(tpu, 1);
    const int CT = chunk * KT;
    const int GC = CT / g;
    const int M = static_cast<int>(c.M);
    const int ssz = w.scale_type == META_F16 ? 2 : 4;
    int xsz = 0;  // bytes of second words per group of 16 rows
    if (bits == 8 && c.path != PATH_SYMMETRIC) xsz = 64;
    else if (bits != 8 && w.zero_mode == ZERO_POINT) xsz = 8;
    else if (bits != 8 && w.zero_mode == ZERO_FLOAT) xsz = 16 * (w.zero_type == META_F16 ? 2 : 4);
    p.chunk_tiles = chunk;
    p.off_stats = align16(M * CT);
    p.off_meta = p.off_stats + align16(12 * M * GC);
    // metadata copies move 4 bytes per lane, whole 256-byte steps
    p.scale_block = (GC * 16 * ssz + 255) / 256 * 256;
    p.x2_block = (GC * xsz + 255) / 256 * 256;
    p.off_x2 = p.off_meta + p.R * p.scale_block;
    p.off_w = p.off_x2 + p.R * p.x2_block;
    p.wave_lds = p.off_w + p.R * chunk * kTileBytes + 16;  // + zero slot
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
    a.off_x2 = p.off_x2;
    a.off_w = p.off_w;
    a.scale_block = p.scale_block;
    a.x2_block = p.x2_block;
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
        else if (dbg && p.R == 2) hipLaunchKernelGGL((skinny_kernel<B, 2, false, Q, ZM, QM, true>), grid, block, lds, stream, a); \
        else if (dbg) hipLaunchKernelGGL((skinny_kernel<B, 1, false, Q, ZM, QM, true>), grid, block, lds, stream, a);    \
        else if (p.R == 2) hipLaunchKernelGGL((skinny_kernel<B, 2, false, Q, ZM, QM, false>), grid, block, lds, stream, a); \
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
