// dot_sinkhorn_forward_noalloc: the Sinkhorn forward with a static device
// scratch instead of a workspace, in a translation unit of its own so that the
// scratch array is a code object of its own.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>
#include <string>

#include "host.hpp"

using namespace dot_amd;

// ---------------------------------------------------------------------------
// Allocation-free forward: the workspace is a file-scope device array.
// ---------------------------------------------------------------------------
// Each GPU this file's code object is loaded on holds its own copy of
// `scratch` until the process ends.  The code object holds no kernel, so the
// HIP runtime (deferred code-object loading, its default) loads it on a
// device only when hipGetSymbolAddress asks for `scratch` there: the first
// call of dot_sinkhorn_forward_noalloc on that device, not any use of the
// library's kernels.  In host code the name `scratch` is not a device
// address: every use goes through the pointer hipGetSymbolAddress returned
// for the device (scratch_on_device).
static __device__ __align__(256) unsigned char scratch[DOT_STATIC_SCRATCH_BYTES];

namespace dot_amd {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};  // device address of `scratch`, per device

// Device address of `scratch` on the device `stream` belongs to, looked up
// once per device with that device current.
int scratch_on_device(hipStream_t stream, void** out) {
    int dev = 0;
    if (stream) {
        hipDevice_t d = 0;
        const hipError_t e = hipStreamGetDevice(stream, &d);
        if (e != hipSuccess) return fail(DOT_ERR_HIP, std::string("hipStreamGetDevice: ") + hipGetErrorString(e));
        dev = int(d);
    } else {
        const hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return fail(DOT_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
    }
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(DOT_ERR_UNSUPPORTED, "device index " + std::to_string(dev) + " out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = 0;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        if (e != hipSuccess) return fail(DOT_ERR_HIP, std::string("hipSetDevice: ") + hipGetErrorString(e));
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p)
            return fail(DOT_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DOT_OK;
}

}  // namespace
}  // namespace dot_amd

using namespace dot_amd;

extern "C" int dot_sinkhorn_forward_noalloc(const dot_sinkhorn_fwd_args* args, dot_stream_t stream_) {
    if (!args) return fail(DOT_ERR_INVALID_ARG, "args is NULL");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    // the workspace without the persistent tier's optional scaled kernel (which
    // the static scratch does not hold: that tier then runs without it)
    const size_t need = forward_workspace_base_bytes(args->B, args->M, args->N, args->max_iter);
    if (need > size_t(DOT_STATIC_SCRATCH_BYTES))
        return fail(DOT_ERR_UNSUPPORTED, "dot_sinkhorn_forward_noalloc: this shape needs " +
                                             std::to_string(need) + " bytes of scratch; the static scratch holds " +
                                             std::to_string(size_t(DOT_STATIC_SCRATCH_BYTES)) +
                                             " (use dot_sinkhorn_forward with a workspace)");
    void* p = nullptr;
    if (int rc = scratch_on_device(stream, &p)) return rc;
    dot_sinkhorn_fwd_args a = *args;
    a.workspace = p;
    a.workspace_bytes = size_t(DOT_STATIC_SCRATCH_BYTES);
    return dot_sinkhorn_forward(&a, stream_);
}
