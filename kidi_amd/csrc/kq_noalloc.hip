// Allocation-free projection entry point (include/kq.h: kq_packed_linear_noalloc).
//
// Callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc) run kq_packed_linear with this file's static device array as the workspace. The array is a
// file-scope __device__ object: every GPU the library runs on holds its own copy, at its own address, until the
// process ends. Host code never passes the array's name to a kernel (on the host it is only a stand-in); the device
// address is looked up once per device with hipGetSymbolAddress and kept in g_scratch_ptr.
//
// Contents: each call leaves the array as its kernels wrote it. Nothing needs clearing between calls, because every
// kernel that reads the workspace (activation codes, block statistics, split-K partial tiles, the GELU temp) writes
// each byte it reads earlier in the same call. Calls on one stream are ordered; calls that overlap on one GPU (from
// several streams) share the array and race.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/kq.h"
#include "kq_internal.hpp"

namespace {

constexpr std::size_t kScratchBytes = std::size_t{64} << 20;  // 64 MiB per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call per device).
kq_status scratch_address(void** out) {
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
        return static_cast<kq_status>(kq::set_error(KQ_RUNTIME, "hipGetDevice failed"));
    if (dev < 0 || dev >= kMaxDevices) return static_cast<kq_status>(kq::set_error(KQ_RUNTIME, "device index out of range"));
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            char msg[160];
            std::snprintf(msg, sizeof msg, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            return static_cast<kq_status>(kq::set_error(KQ_RUNTIME, msg));
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return KQ_OK;
}

}  // namespace

extern "C" {

kq_status kq_packed_linear_noalloc(const kq_weight* weight, const kq_linear_args* args, void* stream) {
    if (!weight || !args) return static_cast<kq_status>(kq::set_error(KQ_INVALID_ARGUMENT, "null weight or arguments"));
    const std::size_t need = kq_linear_workspace_size(weight, args->m);
    if (need > kScratchBytes) {
        char msg[200];
        std::snprintf(msg, sizeof msg,
                      "allocation-free projection needs %zu bytes of scratch, above its static %zu; call kq_packed_linear "
                      "with a workspace",
                      need, kScratchBytes);
        return static_cast<kq_status>(kq::set_error(KQ_INVALID_ARGUMENT, msg));
    }
    kq_linear_args a = *args;
    a.workspace = nullptr;
    a.workspace_bytes = 0;
    if (need) {
        if (kq_status s = scratch_address(&a.workspace); s != KQ_OK) return s;
        a.workspace_bytes = kScratchBytes;
    }
    return kq_packed_linear(weight, &a, stream);
}

}  // extern "C"
