// Host-side helpers shared by the cooperative (one launch, exchange through
// tagged words) kernels of both operators.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>

namespace dot_amd {

// Polls of one exchange word before a cooperative kernel gives up (~1-2 s).
constexpr int kSpinLimit = 1 << 20;

// The poll limit passed to cooperative kernels: kSpinLimit, or the value of
// DOT_AMD_SPIN_LIMIT when set.  A negative value makes every bounded wait
// report a timeout at once (the kernels then finish with NaN outputs and an
// error status); it exists to test the error path.
inline int spin_limit() {
    const char* s = std::getenv("DOT_AMD_SPIN_LIMIT");
    return s && *s ? std::atoi(s) : kSpinLimit;
}

inline int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus;
}

inline int pow2_ceil(int x) {
    int p = 1;
    while (p < x) p *= 2;
    return p;
}

// Launches `kernel` on G workgroups of `threads` threads only if all of them
// can be resident at once (the exchange protocol spins on other workgroups);
// false, with nothing launched, otherwise.
template <class K, class A>
bool launch_cooperative(K kernel, A& args, int G, int threads, size_t lds, hipStream_t stream) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess ||
        per_cu < 1 || int64_t(per_cu) * device_cus() < G)
        return false;
    void* params[] = {&args};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel), dim3(G), dim3(threads), params,
                                      static_cast<unsigned>(lds), stream) == hipSuccess;
}

// Launch of a resident-tier kernel: cooperative when its workgroups wait on
// each other, so that all of them are resident even while other streams run;
// a plain launch when none waits on another (one workgroup per batch element
// and no batch-global test) — a cooperative launch costs ~17 us more.
inline hipError_t launch_grid(const void* kernel, int G, int threads, void** params, size_t lds,
                              hipStream_t stream, bool independent) {
    if (independent) return hipLaunchKernel(kernel, dim3(G), dim3(threads), params, lds, stream);
    return hipLaunchCooperativeKernel(kernel, dim3(G), dim3(threads), params, static_cast<unsigned>(lds), stream);
}

}  // namespace dot_amd
