// Internal types shared by the C ABI (kq_api.cpp) and the kernels (kq_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "kq_layout.hpp"

namespace kq {

enum MetaType : int { META_F32 = 0, META_F16 = 1 };
enum ZeroMode : int { ZERO_NONE = 0, ZERO_POINT = 1, ZERO_FLOAT = 2 };
enum ActType : int { ACT_F32 = 0, ACT_BF16 = 1 };
enum Path : int { PATH_BLOCKWISE = 0, PATH_SYMMETRIC = 1, PATH_PORTABLE = 2 };

// Device-resident packed weight. Either the tiled layout (kq_layout.hpp) or, for group sizes the tiles cannot
// carry, Kidi's own row-major layout.
struct Weight {
    Geometry geo;
    bool tiled = true;
    int scale_type = META_F32;
    int zero_mode = ZERO_NONE;
    int zero_type = META_F32;       // for ZERO_FLOAT
    std::uint8_t* tiles = nullptr;  // tiled codes, or Kidi-layout values [N, K/(8/bits)]
    void* scales = nullptr;         // tiled: [n_tiles][groups_p][16]; row-major: [N][K/g]
    std::uint8_t* zero_points = nullptr;  // ZERO_POINT: tiled [n_tiles][groups_p][8] nibbles; row-major [N][K/g] bytes
    void* zeros = nullptr;          // ZERO_FLOAT: same indexing as scales
    std::int32_t* code_sums = nullptr;  // 8-bit tiled: sum of codes per (row, group), [n_tiles][groups_p][16]
    void* allocation = nullptr;     // one hipMalloc holding all of the above
    std::size_t bytes = 0;
    int device = 0;
    bool scales_positive = false;   // every scale finite and > 0 (LOWBIT_PARITY's precondition)
    // prefill copy for the g = 128 GEMM (kq_gemm8.hip), one more allocation: int8 codes with the zero point folded, in
    // v_mfma_i32_32x32x32_i8 operand order [ceil(N/32)][K/32][64][16], and records [K/128][ceil(N/32)][32] of
    // {s, -1.5 * 2^23 * s, z, 0}
    bool has_prefill = false;
    std::int8_t* prefill_codes = nullptr;
    float* prefill_meta = nullptr;
    void* prefill_alloc = nullptr;
    std::size_t prefill_bytes = 0;
};

// The kernel sequence a projection call runs (kq_debug_route reports it; run_call dispatches on it).
enum Route : int {
    ROUTE_NONE = 0,      // M = 0: nothing runs
    ROUTE_DECODE = 1,    // decode_kernel (kq_decode.hip), activation quantization fused
    ROUTE_SKINNY = 2,    // skinny_kernel (kq_skinny.hip), activation quantization fused
    ROUTE_GEMM_I4 = 3,   // quantize_rows_kernel + gemm_i4_kernel (kq_gemm.hip)
    ROUTE_GEMM_I4G = 4,  // quantize_rows_g_kernel + gemm_i4g_kernel (kq_gemm_g.hip)
    ROUTE_GEMV = 5,      // quantize_kernel + gemv_kernel (kq_kernels.hip)
    ROUTE_GEMM = 6,      // quantize_kernel + gemm_kernel (kq_kernels.hip)
    ROUTE_ROWMAJOR = 7,  // quantize_rowmajor_kernel + rowmajor_kernel (kq_kernels.hip)
    ROUTE_PORTABLE = 8,  // portable_kernel (kq_kernels.hip)
    ROUTE_GEMM8 = 9,     // quantize_rows8_kernel + gemm8_kernel (kq_gemm8.hip)
    ROUTE_GEMM8W = 10    // quantize_rows8_kernel + gemm8w_kernel (kq_gemm8.hip: 128 x 160 tiles, g = 32)
};

// Activation workspace carved out of one device buffer.
struct ActBuffers {
    std::int8_t* q = nullptr;       // [rows_p][cols_p] permuted (tiled) or [M][K] natural (row-major)
    float* scale = nullptr;         // [rows_p][groups_p]
    std::int32_t* sum = nullptr;    // [rows_p][groups_p]
    std::int32_t* zero = nullptr;   // [rows_p][groups_p]
    float* partial = nullptr;       // prefill GEMM with split K: fp32 partial tiles of every K range
    float* gelu_tmp = nullptr;      // [M][N] projection before GELU gating, for gate/up splits inside a row tile
    std::int64_t rows_p = 0;
};

struct LinearCall {
    const Weight* w;
    const void* x;
    int x_type;
    std::int64_t M;
    float input_scale, output_scale;
    float* y;
    int path;
    bool gelu_gate;                 // y [M, N/2] = gelu_tanh(first half) * second half
    bool parity = false;            // LOWBIT_PARITY projection (portable kernel, serial FMA)
    std::int32_t* dump;             // optional int32 partials [M][N][K/g]
    ActBuffers act;
    // optional dumps of the fused (skinny) quantizer: codes [M][K] natural order, block stats [M][K/g]
    std::int8_t* dq_codes = nullptr;
    float* dq_scales = nullptr;
    std::int32_t* dq_sums = nullptr;
    std::int32_t* dq_zeros = nullptr;
    // greedy selection from the decode epilogue: partials [M][workgroups] (kq_greedy.hip), their count per row
    int4* greedy = nullptr;
    int* greedy_parts = nullptr;
    // RMS normalization fused into the activation quantization (decode kernel prologue, prefill row quantizer):
    //   norm 1: the projection input is x * inv(x) * norm_w1
    //   norm 2: h = (norm_res + x * inv(x) * norm_w1) [* norm_scale] (stored to norm_hidden by one workgroup), the
    //           projection input is h * inv(h) * norm_w2
    // norm_inv (prefill): per-row inverse RMS already computed; the quantizer applies x * norm_inv[m] * norm_w1.
    int norm = 0;
    const float* norm_w1 = nullptr;
    const float* norm_w2 = nullptr;
    const void* norm_res = nullptr;
    const float* norm_scale = nullptr;
    float* norm_hidden = nullptr;
    float norm_eps1 = 0.F, norm_eps2 = 0.F;
    const float* norm_inv = nullptr;
};

// RMS normalization kernel (kq_norm.hip): see the modes there.
struct NormLaunch {
    const void* x = nullptr;
    int x_type = ACT_F32;
    const void* residual = nullptr;
    const float* w1 = nullptr;
    const float* scale = nullptr;
    const float* w2 = nullptr;
    float* out1 = nullptr;
    float* out2 = nullptr;
    float* inv_out = nullptr;
    std::int64_t rows = 0, width = 0;
    float eps1 = 0.F, eps2 = 0.F;
};
hipError_t launch_rms_norm(const NormLaunch& n, hipStream_t stream);

// Measurement instrumentation (kq_decode.hip): one launch that only reads `bytes` of `data` once.
hipError_t launch_read_floor(const void* data, std::uint32_t bytes, int* sink, hipStream_t stream);
hipError_t launch_read_floor_shape(const void* data, std::uint32_t bytes, int threads, int loads, bool empty, int* sink,
                                   hipStream_t stream);

// Load-time weight quantization (kq_pack.hip): float weights -> Kidi-layout codes, scales, zeros; error: 1 non-finite
// weight, 2 symmetric scale underflow (OR-ed into *error).
hipError_t launch_pack_weight(const void* w, int dtype, std::int64_t rows, std::int64_t width, int bits, std::int64_t group,
                              bool asym, std::uint8_t* values, float* scales, float* zeros, int* error, hipStream_t stream);

// Launch plan of the skinny (decode, M <= 16) projection with fused activation quantization (kq_skinny.hip).
struct SkinnyPlan {
    int R = 1, W = 1, T = 4;
    int chunk_tiles = 1;
    int wave_lds = 0, off_stats = 0, off_meta = 0, off_x2 = 0, off_w = 0, red_off = 0, lds_bytes = 0;
    int scale_block = 0, x2_block = 0;  // LDS bytes per row tile of a chunk's raw scales and second words
    std::int64_t blocks = 0;
};

bool skinny_plan(const LinearCall& c, SkinnyPlan& p);

// Decode projection for M <= 8 and K a multiple of 512 (at most 8192) with g in {32, 64, 128} (kq_decode.hip).
bool decode_fits(const LinearCall& c);
hipError_t launch_decode(const LinearCall& c, hipStream_t stream);
hipError_t launch_skinny(const LinearCall& c, const SkinnyPlan& p, hipStream_t stream);

// Prefill projection (M > 16) for 4-bit weights with g = 128 and K a multiple of 512 (kq_gemm.hip): a row
// quantizer writing codes [rows_p][K] and transposed block scales [K/128][rows_p] into the workspace, then the int8
// MFMA GEMM. rows_p = round_up(M, 256).
struct GemmPlan {
    int wm = 4, m_blocks = 0, n_blocks = 0, ksplit = 1;
};
GemmPlan gemm_i4_plan(const Weight& w, std::int64_t M, bool gelu);
bool gemm_i4_fits(const LinearCall& c);
hipError_t launch_gemm_i4(const LinearCall& c, const ActBuffers& act, hipStream_t stream);
hipError_t launch_gemm_i4_quantize_dump(const LinearCall& c, const ActBuffers& act, std::int8_t* codes, float* scales,
                                        std::int32_t* sums, std::int32_t* zero_points, hipStream_t stream);

// Prefill projection (M > 16) for 4-bit weights with g = 32 or 64, K a multiple of 128 (kq_gemm_g.hip): a row
// quantizer into c.act (codes [rows_p][K] permuted, block scales [K/g][rows_p]), then a two-stage LDS int8 MFMA GEMM.
bool gemm_i4g_fits(const LinearCall& c);
hipError_t launch_gemm_i4g(const LinearCall& c, hipStream_t stream);
hipError_t launch_gemm_i4g_quantize_dump(const LinearCall& c, std::int8_t* codes, float* scales, std::int32_t* sums,
                                         std::int32_t* zero_points, hipStream_t stream);

// Records `message` as this thread's kq_last_error() and returns `code` (a kq_status value).
int set_error(int code, const char* message);

// Prefill projection (M > 16) for 4-bit weights with g = 128 and K a multiple of 256 from the weight's prefill copy
// (kq_gemm8.hip): a row quantizer into the workspace (codes in the A-operand fragment order, scales [K/128][M_p]),
// then the int8 GEMM on v_mfma_i32_32x32x32_i8 (K split in ranges with a reduction when the grid is small).
struct Gemm8Plan {
    int m_blocks = 0, n_blocks = 0, ksplit = 1;
    int rb = 2;  // 32-row blocks per wave: 2 (256-row tiles) or 1 (128-row tiles, plain g = 128 projections)
    bool wide = false;  // g = 32: 128 x 160 tiles (gemm8w_kernel; n_blocks counts 5-column-block tiles)
};
bool gemm8_eligible(const Weight& w);  // the geometry a prefill copy is built for
Gemm8Plan gemm8_plan(const Weight& w, std::int64_t M, bool gelu);
bool gemm8_fits(const LinearCall& c);
std::size_t gemm8_partial_bytes(const Weight& w, std::int64_t M, bool gelu);
// measurement: one 8-wave workgroup per CU issuing only int8 MFMAs (8 chains x iters per wave); cycles[wg * 8 + wave]
// receives each wave's s_memtime count, sink a value that keeps the MFMAs live
int mfma_ceiling_workgroups();
hipError_t launch_mfma_ceiling(int iters, long long* cycles, int* sink, hipStream_t stream);
// quantize_only: the row quantizer alone (with its parity dumps when d_codes / d_scales / d_sums are set)
hipError_t launch_gemm8(const LinearCall& c, const ActBuffers& act, hipStream_t stream, bool quantize_only = false,
                        std::int8_t* d_codes = nullptr, float* d_scales = nullptr, std::int32_t* d_sums = nullptr);

std::size_t workspace_bytes(const Weight& w, std::int64_t M);
// GELU gating runs after the projection (through ActBuffers::gelu_tmp) only for tiled weights whose gate/up split
// falls inside a 16-row tile; every other path fuses it.
bool gelu_needs_temp(const Weight& w);
ActBuffers carve_workspace(const Weight& w, std::int64_t M, void* base);

// Kernel launchers (kq_kernels.hip). Return hipSuccess or the launch error.
hipError_t launch_quantize(const LinearCall& c, hipStream_t stream);
hipError_t launch_linear(const LinearCall& c, hipStream_t stream);
hipError_t launch_gelu_gate(const float* in, std::int64_t M, std::int64_t I, float* out, hipStream_t stream);
hipError_t launch_gated_multiply(const float* gate, const float* value, std::int64_t n, bool silu, float* out, hipStream_t stream);
hipError_t launch_silu_gate(const float* in, std::int64_t M, std::int64_t I, float* out, hipStream_t stream);

// Greedy token selection (kq_greedy.hip): partials {max, first index, non-finite} per (row, 4096-column chunk) of
// F32 logits, then one token per row from a row's partials in column order (-1 for a non-finite row).
int greedy_chunk_count(std::int64_t width);
hipError_t launch_greedy_chunks(const float* logits, std::int64_t rows, std::int64_t width, int4* parts, hipStream_t stream);
hipError_t launch_greedy_reduce(const int4* parts, std::int64_t rows, int count, std::int32_t* tokens, hipStream_t stream);
hipError_t launch_unpermute_codes(const Weight& w, const ActBuffers& act, std::int64_t M, std::int8_t* codes,
                                  hipStream_t stream);
hipError_t launch_copy_block_stats(const Weight& w, const ActBuffers& act, std::int64_t M, float* scales,
                                   std::int32_t* sums, std::int32_t* zero_points, hipStream_t stream);

// Host-side layout (kq_layout_host.cpp).
void encode_tiles(int bits, std::int64_t rows, std::int64_t cols, const std::uint8_t* values, std::uint8_t* tiles);
void decode_tiles(int bits, std::int64_t rows, std::int64_t cols, const std::uint8_t* tiles, std::int8_t* codes);

}  // namespace kq
