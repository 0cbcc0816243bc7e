/*
 * kq.h — C ABI of the MI355X (gfx950) quantized linear layer: Kidi's PACKED_LINEAR operator.
 *
 * This is the drop-in boundary. Kidi's C++ plugin contract for the operator is
 *   runtime::OperatorBackend::prepare(const OperatorSpec&, TensorInputs) -> unique_ptr<Operator>
 *                                                   (kidi: src/kidi/runtime/operator.h:120-136)
 *   runtime::Operator::run(TensorInputs) / run_into(TensorInputs, span<Tensor>)   (operator.h:106-119)
 * with spec {PACKED_LINEAR, attributes = [bits, group, bit_cast<int32>(output_scale)], epsilon = input_scale}
 * and inputs {x F32 [..., K], W U8 [N, K/(8/bits)], S F32|F16 [N, K/g], (Z F32|F16 [N, K/g])}
 * (src/kidi/ops/context.cpp:933-938, validation :207-218). The entry points below split that contract into
 * load-time weight preparation (kq_weight_pack ~ the CPU backend's one-time tile packing,
 * runtime/ynn/operators.cpp:1061-1089, :2761-2784) and the per-call projection (kq_packed_linear ~
 * Operator::run_into, operators.cpp:1114). No function throws; every one returns a kq_status whose values map
 * 1:1 onto kidi::core::ErrorCode (src/kidi/core/error.h:8-14), with a thread-local message in kq_last_error().
 *
 * Pointers named "device" are HBM addresses on the current HIP device; `stream` is a hipStream_t (NULL = the
 * null stream). Calls are stream-ordered and asynchronous unless stated otherwise.
 */
#ifndef KIDI_AMD_KQ_H
#define KIDI_AMD_KQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kidi::core::ErrorCode + 1 (src/kidi/core/error.h:8-14); KQ_OK has no counterpart (a Result holding a value). */
typedef enum kq_status {
    KQ_OK = 0,
    KQ_INVALID_ARGUMENT = 1,
    KQ_IO = 2,
    KQ_INVALID_MANIFEST = 3,
    KQ_UNSUPPORTED = 4,
    KQ_RUNTIME = 5
} kq_status;

/* Element types at the boundary (subset of kidi::tensor::DType, src/kidi/tensor/dtype.h:10-26), plus
 * KQ_ZP_U8: one unsigned zero-point byte (0..15) per group, meaning the additive zero (8 - zp) * scale that
 * ops::pack_weight stores (src/kidi/ops/quantization.cpp:85). */
typedef enum kq_dtype {
    KQ_NONE = -1,
    KQ_F32 = 0,
    KQ_F16 = 1,
    KQ_BF16 = 2,
    KQ_U8 = 3,
    KQ_I8 = 4,
    KQ_ZP_U8 = 5
} kq_dtype;

typedef enum kq_memory { KQ_HOST = 0, KQ_DEVICE = 1 } kq_memory;

/* Which of Kidi's CPU operators defines the numerics of a call (runtime/ynn/operators.cpp:2739-2900):
 *   KQ_PATH_BLOCKWISE  BlockwiseLinear (:1036-1181): dynamic per-(row, group) int8 activations;
 *   KQ_PATH_SYMMETRIC  SymmetricPackedLinear (:1183-1319): calibrated activations q = rint(x / input_scale);
 *   KQ_PATH_PORTABLE   PortablePackedLinearOp (:2639-2713): float activations, dequantized weights. */
typedef enum kq_path { KQ_PATH_BLOCKWISE = 0, KQ_PATH_SYMMETRIC = 1, KQ_PATH_PORTABLE = 2 } kq_path;

/* A packed weight resident in HBM, re-laid out once for gfx950 (1 KiB tiles of 16 output rows, lane-ordered
 * so one wavefront load instruction moves a whole tile with 16-byte accesses). Immutable after packing. */
typedef struct kq_weight kq_weight;

typedef struct kq_pack_desc {
    int32_t bits;          /* 2, 4 or 8 */
    int32_t group_size;    /* g: cols % g == 0 and g % (8 / bits) == 0 */
    int64_t rows;          /* N (output features) */
    int64_t cols;          /* K (input features) */
    const void* values;    /* Kidi layout: U8 [N, K/(8/bits)], element k in bits (k % (8/bits)) * bits of byte
                              k / (8/bits), two's complement (I8 also accepted for 8-bit) */
    kq_dtype values_dtype; /* KQ_U8 or KQ_I8 */
    const void* scales;    /* [N, K/g] */
    kq_dtype scales_dtype; /* KQ_F32 or KQ_F16 */
    const void* zeros;     /* NULL, or [N, K/g] */
    kq_dtype zeros_dtype;  /* KQ_NONE, KQ_F32 / KQ_F16 (additive zero), or KQ_ZP_U8 (zero-point) */
    kq_memory memory;      /* where values / scales / zeros live */
} kq_pack_desc;

/* Message of the last failed call on this thread ("" if none). */
const char* kq_last_error(void);

/* Library/ABI version and the device architecture it was built for ("gfx950"). */
int32_t kq_version(void);
const char* kq_arch(void);

/* Load-time packing: validate (Context::Impl::run PACKED_LINEAR checks, ops/context.cpp:207-218), re-lay out
 * into the gfx950 tile format on the host and upload to the current device. Synchronous: device sources are read in
 * `stream` order, and a stream under graph capture is refused (KQ_RUNTIME). The source buffers are not retained.
 * Replaces BlockwiseLinear::pack_tiles / SymmetricPackedLinear::pack_tiles
 * (runtime/ynn/operators.cpp:1061-1089, :1206-1231). */
kq_status kq_weight_pack(const kq_pack_desc* desc, void* stream, kq_weight** out);

/* Release a packed weight (device memory is freed after the device finishes queued work). */
void kq_weight_free(kq_weight* weight);

/* Shape of a packed weight. */
kq_status kq_weight_info(const kq_weight* weight, int32_t* bits, int32_t* group_size, int64_t* rows,
                         int64_t* cols, int32_t* has_zeros, size_t* device_bytes);

/* Operator selection for a call (CpuBackend::prepare order, runtime/ynn/operators.cpp:2739-2900;
 * BlockwiseLinear::supports :1038-1059; SymmetricPackedLinear::supports :1185-1204). */
int32_t kq_select_path(int32_t bits, int64_t group_size, int64_t cols, int64_t rows, int32_t has_zeros,
                       float input_scale);

typedef struct kq_linear_args {
    const void* x;          /* device [M, K], row-major */
    kq_dtype x_dtype;       /* KQ_F32 (Kidi's contract, context.cpp:210) or KQ_BF16 */
    int64_t m;              /* M (rows of x); 0 is a no-op */
    float input_scale;      /* OperatorSpec::epsilon: 0 = dynamic activations, > 0 = calibrated */
    float output_scale;     /* bit_cast of attributes[2]: > 0 rounds y to int8 steps of this size */
    float* y;               /* device [M, N] F32 */
    void* workspace;        /* device scratch of kq_linear_workspace_size() bytes, or NULL to use a grow-only
                               buffer the library keeps per (device, stream); it cannot grow while the stream is
                               being captured (KQ_RUNTIME), so captured calls pass a workspace */
    size_t workspace_bytes;
} kq_linear_args;

/* Device bytes of scratch kq_packed_linear needs for M rows (activation codes, block scales and sums). */
size_t kq_linear_workspace_size(const kq_weight* weight, int64_t m);

/* y = PACKED_LINEAR(x; weight) with Kidi's numerics for the selected path: Context::packed_linear
 * (src/kidi/ops/context.cpp:821-939) -> Operator::run_into (runtime/ynn/operators.cpp:1114, :1250, :2667).
 * Asynchronous on `stream`. */
kq_status kq_packed_linear(const kq_weight* weight, const kq_linear_args* args, void* stream);

/* kq_packed_linear without any allocation, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. args->workspace is
 * ignored: the workspace is a static device array of the library (64 MiB per device, held until the process ends),
 * and a call whose kq_linear_workspace_size() exceeds it returns KQ_INVALID_ARGUMENT without running. Calls on one
 * stream are ordered; calls that overlap on one device (several streams) share the array and race. Results equal
 * kq_packed_linear's. */
kq_status kq_packed_linear_noalloc(const kq_weight* weight, const kq_linear_args* args, void* stream);

/* Fused projections that share one activation read (Kidi fuses gate+up and k+v by concatenating rows,
 * model/gemma4.cpp:308-322; its CUDA backend groups projections with one input, runtime/cuda/operators.cpp:366-437):
 * kq_weight_pack_concat packs `count` weights with equal bits, group and K into one weight whose rows are the
 * concatenation in order (e.g. fused QKV). Synchronous. */
kq_status kq_weight_pack_concat(const kq_pack_desc* descs, int32_t count, void* stream, kq_weight** out);

/* Gate/up projection fused with GELU-tanh gating: `weight` holds [gate rows; up rows] (2*I rows, as Kidi's
 * gate_up_proj, model/gemma4.cpp:308-316); y [M, I] = gelu_tanh(x W_gate^T) * (x W_up^T)
 * (Context::gelu_gate, ops/context.cpp:957-963; formula eager_test.cpp:444-452). */
kq_status kq_packed_linear_gelu_gate(const kq_weight* weight, const kq_linear_args* args, void* stream);

/* Kidi's LOWBIT_PARITY projection: runtime::parity::packed_linear (src/kidi/runtime/parity_math.cpp:226-291), which
 * Context::packed_linear runs instead of PACKED_LINEAR under InferencePrecision::LOWBIT_PARITY (ops/context.cpp:917-932).
 * Activations rounded to the calibration grid, clamp(nearbyint(x / input_scale), -128, 127) * input_scale; weights
 * dequantized to c * s (zeros bound to the weight are not applied, as in the reference); each output one fused
 * multiply-add per column in column order; the result rounded to the output_scale grid. Outside the reference's domain
 * (x not F32, input_scale or output_scale not > 0, F16 scales, dimensions above INT32_MAX) it returns KQ_UNSUPPORTED
 * with the reference's message, and KQ_INVALID_ARGUMENT when a scale is not finite and positive. The serial form is
 * the reference's for M < 8; for M >= 8 the reference sums with Accelerate's sgemm (its order is not reproduced).
 * Asynchronous on `stream`; no workspace. */
kq_status kq_lowbit_parity_linear(const kq_weight* weight, const kq_linear_args* args, void* stream);

/* Operation::GELU_MULTIPLY / SILU_MULTIPLY: y = act(gate) * value element by element over `count` F32 values of two
 * tensors of one shape (Context::gelu_multiply / silu_multiply, src/kidi/ops/context.cpp:944-957; GatedMultiplyOp,
 * runtime/ynn/operators.cpp:267-311), the slice form of the gated feed-forward (layers/gemma4.cpp:213-225) with the
 * expressions of kq_packed_linear_gelu_gate's gating (GELU-tanh) and the SiLU gate. Device pointers; `y` may be `gate`
 * or `value` (in place); asynchronous on `stream`. */
kq_status kq_gelu_multiply(const float* gate, const float* value, int64_t count, float* y, void* stream);
kq_status kq_silu_multiply(const float* gate, const float* value, int64_t count, float* y, void* stream);

/* Gated feed-forward of one decoder layer: Context::gated_feed_forward (src/kidi/ops/context.cpp:970-996) ->
 * Operation::GATED_FEED_FORWARD, run by PackedFeedForward (runtime/ynn/operators.cpp:1321-1517) for calibrated
 * inputs. `gate_up` holds [gate rows; up rows] (2*I rows, K columns), `down` holds K rows of I columns, equal bits.
 *   h [M, I] = act(gate) * up, where [gate | up] is the gate/up projection of x with gate_up_input_scale and
 *              gate_up_output_scale, act = GELU-tanh or (silu != 0, attributes[6]) SiLU;
 *   y [M, K] = the down projection of h with down_input_scale (h's int8 codes clamp(rint(h / down_input_scale)),
 *              PackedFeedForward's mid tiles) and down_output_scale.
 * Zero input scales select dynamic activations, as the composed form Context::gated_feed_forward runs outside
 * CHECKPOINT precision (:977-984). Asynchronous on `stream`. */
typedef struct kq_ffn_args {
    const void* x;              /* device [M, K] */
    kq_dtype x_dtype;           /* KQ_F32 or KQ_BF16 */
    int64_t m;
    float gate_up_input_scale;  /* OperatorSpec::epsilon */
    float gate_up_output_scale; /* bit_cast of attributes[3] */
    float down_input_scale;     /* attributes[4] */
    float down_output_scale;    /* attributes[5] */
    int32_t silu;               /* attributes[6] */
    float* y;                   /* device [M, K] F32 */
    void* workspace;            /* device scratch of kq_ffn_workspace_size() bytes, or NULL (library buffer) */
    size_t workspace_bytes;
} kq_ffn_args;

size_t kq_ffn_workspace_size(const kq_weight* gate_up, const kq_weight* down, int64_t m);
kq_status kq_gated_feed_forward(const kq_weight* gate_up, const kq_weight* down, const kq_ffn_args* args, void* stream);

/* Greedy token: GREEDY_TOKEN (GreedyToken, runtime/ynn/operators.cpp:117-178; Context::greedy_token). tokens[r]
 * is the first index of the maximum of row r of logits [rows, width] (device F32), or -1 when the row holds a NaN or
 * an infinity (tests/kidi/layers/eager_test.cpp:231-252). tokens: device I32 [rows]. width must be positive. */
size_t kq_greedy_workspace_size(int64_t rows, int64_t width);
kq_status kq_greedy_token(const float* logits, int64_t rows, int64_t width, int32_t* tokens, void* workspace,
                          size_t workspace_bytes, void* stream);

/* The output head fused with greedy selection (the step after the head, Context::greedy_token on
 * Context::packed_linear's logits): tokens [M] (device I32) of the projection kq_packed_linear computes. args->y
 * may be NULL (the logits are then not stored). For decode shapes (M <= 8) each workgroup of the projection reduces
 * its logits on chip; other shapes compute the logits, then select. args->workspace, when given, must hold
 * kq_greedy_linear_workspace_size() bytes. No counterpart call exists in the reference; it composes the two ops. */
size_t kq_greedy_linear_workspace_size(const kq_weight* weight, int64_t m);
kq_status kq_packed_linear_greedy(const kq_weight* weight, const kq_linear_args* args, int32_t* tokens, void* stream);

/* Load-time weight quantization on the device: ops::pack_weight (src/kidi/ops/quantization.cpp:12-133), the step
 * Context::prepare_linear_weights runs for float weights (src/kidi/ops/context.cpp:783-812) before they reach
 * PACKED_LINEAR. weight: device [rows, cols] F32 | F16 | BF16. Outputs (device, Kidi layout, ready for
 * kq_weight_pack with memory = KQ_DEVICE): values U8 [rows, cols / (8 / bits)], scales F32 [rows, cols / g] and, when
 * asymmetric_clip and bits == 4, zeros F32 [rows, cols / g] (the additive zero (8 - zp) * scale; zeros may be NULL
 * otherwise). Symmetric: scale = max|w| / (2^(bits-1) - 1), codes rounded half away from zero; asymmetric 4-bit: the
 * 11-step MSE clip. Non-finite weights and a scale that underflows return KQ_INVALID_ARGUMENT. Synchronous (a stream
 * under graph capture is refused); the error flag it reads back is per (device, stream), so concurrent calls on one
 * stream from several threads are not supported. */
kq_status kq_quantize_weight(const void* weight, kq_dtype dtype, int64_t rows, int64_t cols, int32_t bits,
                             int32_t group_size, int32_t asymmetric_clip, uint8_t* values, float* scales, float* zeros,
                             void* stream);

/* RMS normalization over the last axis: RMS_NORM / RMS_NORM_RESIDUAL (Context::rms_norm and
 * Context::rms_norm_residual, src/kidi/ops/context.cpp:1043-1049, :1103-1122; the CPU RmsNorm operator,
 * runtime/ynn/operators.cpp:553-620):
 *   plain:    y[r, i] = x[r, i] * inv_r * weight[i]
 *   residual: y[r, i] = (residual[r, i] + x[r, i] * inv_r * weight[i]) * output_scale   (no scaling when NULL)
 * with inv_r = 1 / sqrt(sum_i x[r, i]^2 / width + epsilon); epsilon must be finite and > 0 (context.cpp:1108). The
 * sum of squares has one fixed order in this library (8-column pieces in column order, a pairwise tree over the 64
 * pieces of each 512-column segment, segments in order), shared by the fused projection below. */
typedef struct kq_rms_args {
    const void* x;             /* device [rows, width] */
    kq_dtype x_dtype;          /* KQ_F32 or KQ_BF16 */
    int64_t rows;
    int64_t width;
    const float* weight;       /* device F32 [width] */
    const void* residual;      /* NULL (RMS_NORM) or device [rows, width] of x_dtype (RMS_NORM_RESIDUAL) */
    const float* output_scale; /* NULL or device F32 [1]; residual form only (the layer scalar, layers/gemma4.cpp:416) */
    float epsilon;
    float* y;                  /* device F32 [rows, width] */
} kq_rms_args;
kq_status kq_rms_norm(const kq_rms_args* args, void* stream);

/* A projection of an RMS-normalized input, the normalization fused into the activation quantization: Kidi's
 * decoder layer runs Context::rms_norm right before each projection group (input_layernorm before q_proj/kv_proj,
 * pre_feedforward_layernorm before gate_up_proj, src/kidi/layers/gemma4.cpp:405, :410-413), and before that norm the
 * residual add of the previous block (post_attention_layernorm's rms_norm_residual, :407). With `residual` NULL:
 *   y = PACKED_LINEAR(rms_norm(x; weight, epsilon))
 * With `residual` set (the residual chain of gemma4.cpp:407-410):
 *   hidden = rms_norm_residual(x; residual_weight, residual, residual_epsilon, residual_scale)   (stored to `hidden`)
 *   y      = PACKED_LINEAR(rms_norm(hidden; weight, epsilon))
 * gelu_gate != 0 applies kq_packed_linear_gelu_gate's gating. Decode shapes (M <= 8, K <= 2048, 16-byte aligned norm
 * operands) run as one launch; the prefill path computes per-row statistics, then quantizes normalized rows; other
 * shapes normalize into the workspace first. Every path yields the bits of kq_rms_norm followed by the projection.
 * args->workspace, when given, must hold kq_rms_linear_workspace_size() bytes. */
typedef struct kq_norm_desc {
    const float* weight;          /* device F32 [K]: the norm weight of the projection input */
    float epsilon;
    const void* residual;         /* NULL, or device [M, K] of args->x_dtype */
    const float* residual_weight; /* device F32 [K] (residual form) */
    const float* residual_scale;  /* NULL or device F32 [1] (residual form) */
    float residual_epsilon;
    float* hidden;                /* device F32 [M, K]: receives hidden (residual form) */
} kq_norm_desc;
size_t kq_rms_linear_workspace_size(const kq_weight* weight, int64_t m);
kq_status kq_packed_linear_rms(const kq_weight* weight, const kq_linear_args* args, const kq_norm_desc* norm,
                               int32_t gelu_gate, void* stream);

/* Persisted gfx950 layout, the role of Kidi's packed-operator cache (runtime/ynn/feed_forward_cache.h:11-38,
 * feed_forward_cache.cpp): a packed weight as one host blob (header + the device image) and back, so a later load
 * skips validation and re-layout. The blob holds the layout version and the weight's geometry; kq_weight_import
 * rejects with KQ_INVALID_MANIFEST, before any device call, a blob of another version, of the wrong size, or whose
 * header (shape, modes, offsets, image size) differs from the image this library builds for that geometry and those
 * modes. Both calls are synchronous and refuse a stream under graph capture. */
size_t kq_weight_export_size(const kq_weight* weight);
kq_status kq_weight_export(const kq_weight* weight, void* host, size_t bytes, void* stream);
kq_status kq_weight_import(const void* host, size_t bytes, void* stream, kq_weight** out);

/* ---- parity instrumentation (same kernels as kq_packed_linear, with an extra store) --------------------- */

/* Activation quantization exactly as the projection performs it: codes int8 [M, K] (natural k order),
 * scales f32 [M, K/g], sums int32 [M, K/g] (sum of codes per block), zero_points int32 [M, K/g] (0 unless the
 * 8-bit dynamic form). All outputs are device pointers. */
kq_status kq_debug_quantize(const kq_weight* weight, const void* x, kq_dtype x_dtype, int64_t m, float input_scale,
                            int8_t* codes, float* scales, int32_t* sums, int32_t* zero_points, void* stream);

/* Runs the projection kernel that kq_packed_linear would run for these arguments and also writes its int32
 * per-group partials [M, N, K/g]: sum over the group of x_code * w_code, where w_code = c (symmetric), u - zp
 * (ZP_U8 zero-points, u = c + 8) or c (additive float zeros), and x_code = q - zp_a for 8-bit dynamic. (Where
 * kq_packed_linear takes route 10, g = 32 in 128 x 160 tiles, the dump comes from the 256 x 128 instance of the same
 * GEMM, route 9, whose y is bit-identical: the same operations per element in the same order.) */
kq_status kq_debug_partials(const kq_weight* weight, const kq_linear_args* args, int32_t* partials, void* stream);

/* The kernel sequence a projection call takes, without running it (no counterpart in the reference; for tests that
 * assert which kernels they cover): 0 none (M = 0), 1 decode_kernel, 2 skinny_kernel, 3 quantize_rows_kernel +
 * gemm_i4_kernel, 4 quantize_rows_g_kernel + gemm_i4g_kernel, 5 quantize_kernel + gemv_kernel, 6 quantize_kernel +
 * gemm_kernel, 7 quantize_rowmajor_kernel + rowmajor_kernel, 8 portable_kernel, 9 quantize_rows8_kernel + gemm8_kernel
 * (from the weight's prefill copy), 10 quantize_rows8_kernel + gemm8w_kernel (the same copy, g = 32 in 128 x 160
 * tiles where 256 x 128 tiles leave compute units idle); -1 for invalid arguments.
 * kq_debug_route_shape answers for a weight described by its geometry and modes (zero_mode: 0 none, 1 ZP_U8 zero
 * points or additive zeros equal to (8 - zp) * scale, 2 other additive zeros) and touches no device. */
int32_t kq_debug_route(const kq_weight* weight, const kq_linear_args* args, int32_t gelu_gate);
int32_t kq_debug_route_shape(int32_t bits, int32_t group_size, int64_t rows, int64_t cols, int32_t zero_mode,
                             int32_t scale_f16, int64_t m, kq_dtype x_dtype, float input_scale, int32_t gelu_gate);

/* ---- measurement instrumentation (no counterpart in the reference) ----------------------------------------- */

/* One launch that only reads `bytes` (a multiple of 16, at most 2 GiB) of device memory once (512-lane workgroups,
 * one 16-byte load per lane: the fastest geometry of kq_debug_read_floor_shape's sweep on MI355X; arguments
 * preloaded as the decode kernel's); `sink` is a device int32 it writes only by chance. Its per-launch time is the
 * floor of any single-launch kernel that streams a buffer of that size. */
kq_status kq_debug_read_floor(const void* data, size_t bytes, int32_t* sink, void* stream);
/* The same read at a chosen launch geometry: `threads` per workgroup (64, 128, 256, 512 or 1024), `loads` 16-byte
 * loads per lane (1, 2, 4, 8 or 16), ceil(bytes / (16 threads loads)) workgroups; with `empty` nonzero an empty
 * kernel of that grid instead (the launch cost alone). */
kq_status kq_debug_read_floor_shape(const void* data, size_t bytes, int32_t threads, int32_t loads, int32_t empty,
                                    int32_t* sink, void* stream);

/* The sustained int8 MFMA rate of the device: one launch of kq_debug_mfma_ceiling_workgroups() workgroups (one per
 * compute unit) of 8 waves, as the prefill GEMM, each wave issuing `iterations` (1 to 2^24) rounds of eight
 * independent v_mfma_i32_32x32x32_i8 (65,536 int8 operations each) and nothing else. `cycles` (device, one int64 per
 * wave: workgroups x 8) receives each wave's s_memtime count over its loop (a timestamp counter, not the shader
 * clock), `sink` (device, int32, same count) a value that keeps the MFMAs live. Operations per launch: workgroups x 8
 * x iterations x 8 x 65,536; the rate follows from the launch's device time. */
int32_t kq_debug_mfma_ceiling_workgroups(void);
kq_status kq_debug_mfma_ceiling(int32_t iterations, int64_t* cycles, int32_t* sink, void* stream);

/* Host-only (no GPU): the gfx950 tile layout of a Kidi-layout weight and its inverse, for layout tests. */
size_t kq_layout_bytes(int32_t bits, int32_t group_size, int64_t rows, int64_t cols);
kq_status kq_layout_encode_host(int32_t bits, int64_t rows, int64_t cols, const uint8_t* values, uint8_t* tiles);
kq_status kq_layout_decode_host(int32_t bits, int64_t rows, int64_t cols, const uint8_t* tiles, int8_t* codes);

#ifdef __cplusplus
}
#endif

#endif /* KIDI_AMD_KQ_H */
