// nnops_hip_gemm_i8_noalloc: the integer GEMM entry point for callers that
// cannot allocate (code under HIP graph capture, serving loops, harnesses
// that forbid hipMalloc). It runs exactly nnops_hip_gemm_i8's kernels, with
// their workspace (staged transposed operands, compensation sums, K-split
// partials) taken from a fixed device array instead of the caller.
//
// The array lives in this code object: each GPU the library runs on holds its
// own copy, kScratchBytes of device memory, until the process ends. Its
// address on a device is looked up once, with that device current, by
// hipGetSymbolAddress; host code only ever passes that address to the
// kernels (the array's name is a host-side stand-in, not a device address).
// Calls on one GPU share the array: two calls that may overlap on one GPU
// (different streams, or another thread) race. nnops_hip_gemm_i8 needs no
// zeroed workspace, so nothing is cleared between calls.
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.hpp"
#include "nnops_amd.h"

namespace {

constexpr size_t kScratchBytes = NNOPS_HIP_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `dev` (the current device), looked up on the
// first call there; nullptr if the lookup fails.
void* scratch_on(int dev)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        // The first call on a device may come while the caller's stream is
        // being captured into a graph: the lookup enqueues nothing, so this
        // thread's capture mode is relaxed around it (a global-mode capture
        // would otherwise reject an API call it cannot vet) and restored.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        const bool exchanged = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
        void* p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (exchanged) {
            (void)hipThreadExchangeStreamCaptureMode(&mode);
        }
        if (rc != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int nnops_hip_gemm_i8_noalloc(const NnopsGemmI8Args* args, void* stream)
{
    const nnops_amd::TimingDisarm disarm;
    if (args == nullptr) {
        return NNOPS_INVALID_ARGUMENT;
    }
    const size_t need = nnops_hip_gemm_i8_workspace_size(args);
    if (need > kScratchBytes) {
        return NNOPS_OUT_OF_MEMORY;   // the plan needs more than the fixed array holds
    }
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return NNOPS_INTERNAL;
    }
    if (stream != nullptr) {
        int sdev = -1;
        if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess) {
            (void)hipGetLastError();
            return NNOPS_INVALID_ARGUMENT;
        }
        if (sdev != dev) {
            return NNOPS_INVALID_ARGUMENT;   // the scratch of the current device would be used on another
        }
    }
    void* ws = need > 0 ? scratch_on(dev) : nullptr;
    if (need > 0 && ws == nullptr) {
        return NNOPS_INTERNAL;
    }
    return nnops_hip_gemm_i8(args, ws, need > 0 ? kScratchBytes : 0, stream);
}
