// Host-side helpers shared by the one-launch kernels of both operators whose
// workgroups exchange values through tagged words (resident and persistent
// tiers, one-pass bidirectional softmax).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>

namespace dot_amd {

// Polls of one exchange word before a kernel of the exchange tiers gives up
// (~2-4 s: long enough for work of other libraries that holds CUs to finish).
constexpr int kSpinLimit = 1 << 22;

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

// 1 when exchange stores may stop in the writer's XCD L2 for readers on the
// same XCD (workgroup-scope stores read by agent-scope loads, a behaviour of
// the L2 measured on gfx950 and checked per launch by the XCC ids the
// workgroups announce), 0 to keep every exchange store at agent scope: on
// devices other than gfx950, and with DOT_AMD_AGENT_SCOPE=1.
inline int local_exchange_allowed() {
    const char* e = std::getenv("DOT_AMD_AGENT_SCOPE");
    if (e && e[0] == '1') return 0;
    static std::atomic<int> known[64];  // per device: 0 unknown, 1 gfx950, 2 other
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int k = known[dev].load(std::memory_order_relaxed);
    if (k == 0) {
        hipDeviceProp_t prop;
        k = (hipGetDeviceProperties(&prop, dev) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0)
                ? 1 : 2;
        known[dev].store(k, std::memory_order_relaxed);
    }
    return k == 1 ? 1 : 0;
}

inline int pow2_ceil(int x) {
    int p = 1;
    while (p < x) p *= 2;
    return p;
}

// Launch of a resident-tier kernel.  Its workgroups wait on one another
// (unless `independent`: one workgroup per batch element and no batch-global
// test), so all G of them must be resident at once.  G never exceeds the
// device's resident capacity for the kernel (the callers check occupancy), so
// a plain launch has them all resident as soon as the CUs are free; a
// cooperative launch adds a device-wide order among such launches and costs
// ~18 us more per launch (two per Sinkhorn fwd+bwd step: 5 % of a C3 step).
// The order that matters here -- two of this library's exchange kernels never
// sharing the device, so neither holds CUs the other's missing workgroups
// need -- is kept by resident_order: a launch on a stream other than the
// previous launch's first waits for that launch.  Work of other libraries
// that holds CUs (a communication kernel on a side stream) only delays the
// missing workgroups; the waits are bounded (spin_limit) and a wait that gives
// up is reported as an error, never as a result.  DOT_AMD_COOPERATIVE=1 asks
// for cooperative launches instead (a device shared with long-running
// kernels of other processes).
inline bool cooperative_requested() {
    const char* s = std::getenv("DOT_AMD_COOPERATIVE");
    return s && s[0] == '1';
}

class ResidentOrder {
  public:
    // Plain launch of `kernel`, after the previous one of this device when that
    // went to another stream.  The launch itself marks its completion on an
    // event (hipExtLaunchKernel's stop event: no separate marker in the queue).
    hipError_t launch(const void* kernel, int G, int threads, void** params, size_t lds, hipStream_t stream,
                      bool cooperative = false) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
        while (flag_.test_and_set(std::memory_order_acquire)) {
        }
        Slot& s = slots_[dev];
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        // a capture cannot wait on (or record) work outside it
        const bool capturing = hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
        hipError_t e = hipSuccess;
        if (!capturing && s.ev && s.last != stream) e = hipStreamWaitEvent(stream, s.ev, 0);
        if (!capturing && !s.ev && hipEventCreateWithFlags(&s.ev, hipEventDefault) != hipSuccess) s.ev = nullptr;
        if (e == hipSuccess && cooperative) {
            e = hipLaunchCooperativeKernel(kernel, dim3(G), dim3(threads), params, static_cast<unsigned>(lds),
                                           stream);
            if (e == hipSuccess && !capturing && s.ev && hipEventRecord(s.ev, stream) == hipSuccess) s.last = stream;
        } else if (e == hipSuccess) {
            e = hipExtLaunchKernel(kernel, dim3(G), dim3(threads), params, lds, stream, nullptr,
                                   capturing ? nullptr : s.ev, 0);
            if (e == hipSuccess && !capturing && s.ev) s.last = stream;
        }
        flag_.clear(std::memory_order_release);
        return e;
    }

  private:
    static constexpr int kMaxDevices = 64;
    struct Slot {
        hipEvent_t ev = nullptr;  // completes with the device's last launch (never destroyed)
        hipStream_t last = nullptr;
    };
    Slot slots_[kMaxDevices];
    std::atomic_flag flag_ = ATOMIC_FLAG_INIT;
};

inline ResidentOrder& resident_order() {
    static ResidentOrder* o = new ResidentOrder();  // never destroyed: its events outlive static teardown
    return *o;
}

inline hipError_t launch_grid(const void* kernel, int G, int threads, void** params, size_t lds,
                              hipStream_t stream, bool independent) {
    if (independent) return hipLaunchKernel(kernel, dim3(G), dim3(threads), params, lds, stream);
    return resident_order().launch(kernel, G, threads, params, lds, stream, cooperative_requested());
}

// Launch of a persistent-tier kernel (workgroups that wait on one another,
// milliseconds long): only if all G workgroups can be resident at once
// (false, with nothing launched, otherwise).  Launched as the resident tier's
// kernels are: plainly, in resident_order, cooperative only when
// DOT_AMD_COOPERATIVE=1.
template <class K, class A>
bool launch_persistent(K kernel, A& args, int G, int threads, size_t lds, hipStream_t stream) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess ||
        per_cu < 1 || int64_t(per_cu) * device_cus() < G)
        return false;
    void* params[] = {&args};
    return resident_order().launch(reinterpret_cast<const void*>(kernel), G, threads, params, lds, stream,
                                   cooperative_requested()) == hipSuccess;
}

}  // namespace dot_amd
