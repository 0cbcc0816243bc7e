// Greedy token selection (Kidi's GREEDY_TOKEN: GreedyToken, runtime/ynn/operators.cpp:117-178; Context::greedy_token):
// per row of F32 logits, the first index of the maximum, or -1 when the row holds a NaN or an infinity (the KAT of
// tests/kidi/layers/eager_test.cpp:231-252: ties go to the lower index, -0 equals 0, +inf / -inf / NaN give -1).
//
// Two passes, both deterministic:
//   greedy_chunks_kernel: one workgroup per (row, 4096-column chunk) writes a partial {max, first index, non-finite};
//     the head projection's decode kernel writes the same partials from its epilogue (one per workgroup) instead,
//     so the logits need not be stored.
//   greedy_reduce_kernel: one workgroup per row combines its partials in column order.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "kq_internal.hpp"

namespace kq {
namespace {

constexpr int kChunk = 4096;  // columns per stage-1 workgroup (256 threads x 16)

struct Best {
    float v;
    int n;
    int bad;
};

// the better of two candidates: larger value, then lower index (NaN never wins; it is flagged instead)
__device__ __forceinline__ Best better(Best a, Best b) {
    Best r = (b.v > a.v || (b.v == a.v && b.n < a.n)) ? b : a;
    r.bad = a.bad | b.bad;
    return r;
}

__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        Best o;
        o.v = __shfl_xor(b.v, off);
        o.n = __shfl_xor(b.n, off);
        o.bad = __shfl_xor(b.bad, off);
        b = better(b, o);
    }
    return b;
}

__device__ __forceinline__ Best block_best(Best b, Best* sh) {
    b = wave_best(b);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    if (lane == 0) sh[wave] = b;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < waves; ++w) b = better(b, sh[w]);
    return b;  // valid in thread 0
}

__global__ __launch_bounds__(256) void greedy_chunks_kernel(const float* logits, std::int64_t width, int chunks, int4* parts) {
    __shared__ Best sh[4];
    const std::int64_t row = blockIdx.y;
    const std::int64_t base = static_cast<std::int64_t>(blockIdx.x) * kChunk;
    const float* p = logits + row * width;
    Best b{-__builtin_inff(), INT_MAX, 0};
#pragma unroll 4
    for (int j = 0; j < kChunk / 256; ++j) {
        const std::int64_t n = base + j * 256 + threadIdx.x;
        if (n < width) {
            const float v = p[n];
            if (!__builtin_isfinite(v)) b.bad = 1;
            else if (v > b.v) {  // the thread visits its columns in increasing order: strict > keeps the first
                b.v = v;
                b.n = static_cast<int>(n);
            }
        }
    }
    b = block_best(b, sh);
    if (threadIdx.x == 0) parts[row * chunks + blockIdx.x] = make_int4(__float_as_int(b.v), b.n, b.bad, 0);
}

__global__ __launch_bounds__(256) void greedy_reduce_kernel(const int4* parts, int count, std::int32_t* tokens) {
    __shared__ Best sh[4];
    const int row = blockIdx.x;
    Best b{-__builtin_inff(), INT_MAX, 0};
    for (int i = threadIdx.x; i < count; i += blockDim.x) {  // partials cover increasing column ranges
        const int4 q = parts[static_cast<std::int64_t>(row) * count + i];
        b = better(b, Best{__int_as_float(q.x), q.y, q.z});
    }
    b = block_best(b, sh);
    if (threadIdx.x == 0) tokens[row] = (b.bad || b.n == INT_MAX) ? -1 : b.n;
}

}  // namespace

int greedy_chunk_count(std::int64_t width) { return static_cast<int>((width + kChunk - 1) / kChunk); }

hipError_t launch_greedy_chunks(const float* logits, std::int64_t rows, std::int64_t width, int4* parts, hipStream_t stream) {
    const int chunks = greedy_chunk_count(width);
    hipLaunchKernelGGL(greedy_chunks_kernel, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)), dim3(256), 0,
                       stream, logits, width, chunks, parts);
    return hipGetLastError();
}

hipError_t launch_greedy_reduce(const int4* parts, std::int64_t rows, int count, std::int32_t* tokens, hipStream_t stream) {
    hipLaunchKernelGGL(greedy_reduce_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, parts, count, tokens);
    return hipGetLastError();
}

}  // namespace kq
