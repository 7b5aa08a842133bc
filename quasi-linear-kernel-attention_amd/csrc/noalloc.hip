// Allocation-free Laplace forward: qlka_laplace_fwd over a workspace that lives in this file's static device array,
// for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). The caller passes inputs and outputs only; nothing here calls hipMalloc / hipFree.
//
// The array is `scratch` below, SCRATCH_BYTES on every device the library runs on, held until the process ends. Host
// code never passes `scratch` itself to a kernel (in host code that name is only a stand-in for the symbol): the first
// call on a device, with that device current, looks up the array's device address with hipGetSymbolAddress and keeps
// it per device; every call on that device then hands that address to qlka_laplace_fwd as its workspace.
//
// Every call on a device shares that device's array and leaves its contents behind. No stage of the Laplace forward
// reads workspace memory before writing it in the same call, so nothing needs clearing between calls; calls that
// overlap in time on one device (e.g. from two streams) would race on the array and must be serialised by the caller.
#include "qlka.h"
#include "qlka_internal.h"

#include <cstdio>
#include <mutex>

// 512 MiB: a Laplace forward needs about 310 MB of workspace per p at N = M = 16384, D = C = 64, so this holds one p
// there (the call then runs one p at a time); shapes whose single-p workspace exceeds it are refused.
constexpr size_t SCRATCH_BYTES = size_t(512) << 20;
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_scratch[MAX_DEVICES];     // device address of `scratch` on each device, looked up once with it current

int scratch_address(int dev, void** out) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace

extern "C" int qlka_laplace_fwd_noalloc(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                                        int P, int D, int N, int M, int C, void* stream) {
    if (int e = qlka::validate_dims(P, D, N, M, C)) return e;
    const size_t one_p = qlka::laplace_fwd_chunk_ws(1, D, N, M, C);
    if (one_p > SCRATCH_BYTES) {
        char msg[256];
        snprintf(msg, sizeof(msg), "the workspace of one p (%zu bytes for D=%d, N=%d, M=%d, C=%d) exceeds the %zu-byte "
                 "static scratch of qlka_laplace_fwd_noalloc; use qlka_laplace_fwd with a workspace", one_p, D, N, M,
                 C, SCRATCH_BYTES);
        return qlka::report_error(QLKA_EINVAL, msg);
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
        return qlka::report_error(QLKA_EHIP, "qlka_laplace_fwd_noalloc: no usable current device");
    hipStream_t st = (hipStream_t)stream;
    if (st != nullptr) {
        int sdev = dev;
        if (hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev)
            return qlka::report_error(QLKA_EINVAL, "qlka_laplace_fwd_noalloc: the stream must belong to the current "
                                                   "device");
    }
    void* ws = nullptr;
    if (int e = scratch_address(dev, &ws)) {
        char msg[256];
        snprintf(msg, sizeof(msg), "qlka_laplace_fwd_noalloc: hipGetSymbolAddress(scratch): %s",
                 hipGetErrorString((hipError_t)e));
        return qlka::report_error(QLKA_EHIP, msg);
    }
    return qlka_laplace_fwd(q, k, v, out_w, out_u, P, D, N, M, C, ws, SCRATCH_BYTES, stream);
}
