// Host-side helpers for the C ABI: thread-local error text, launch checking,
// workspace carving and the optional per-kernel event profiler.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <string>

#include "../../include/dot_amd.h"

namespace dot_amd {

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Clears this thread's last error and returns DOT_OK.
int ok();

// Checks hipGetLastError() after a launch; returns DOT_OK or DOT_ERR_HIP.
int check_launch(const char* what);

// Bump allocator over a caller-provided workspace; every carve is 256-byte aligned.
class Carver {
  public:
    explicit Carver(void* base) : base_(static_cast<char*>(base)), off_(0) {}
    template <class T>
    T* take(size_t count) {
        off_ = (off_ + 255) & ~size_t(255);
        T* p = base_ ? reinterpret_cast<T*>(base_ + off_) : nullptr;
        off_ += count * sizeof(T);
        return p;
    }
    size_t used() const { return (off_ + 255) & ~size_t(255); }

  private:
    char* base_;
    size_t off_;
};

// Event profiler.  When enabled, `ProfScope` brackets a launch with two events
// on the launch stream; dot_profile_collect() folds finished pairs into
// per-kernel totals.
bool profiling_enabled(const char* name);
void profile_push(const char* name, hipEvent_t start, hipEvent_t stop);
hipEvent_t profile_event();

class ProfScope {
  public:
    ProfScope(const char* name, hipStream_t stream) : name_(name), stream_(stream) {
        if (profiling_enabled(name)) {
            start_ = profile_event();
            stop_ = profile_event();
            (void)hipEventRecord(start_, stream_);
        }
    }
    ~ProfScope() {
        if (start_) {
            (void)hipEventRecord(stop_, stream_);
            profile_push(name_, start_, stop_);
        }
    }
    ProfScope(const ProfScope&) = delete;
    ProfScope& operator=(const ProfScope&) = delete;

  private:
    const char* name_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
    hipEvent_t stop_ = nullptr;
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rows per workgroup strip of a streaming sweep: the largest power of two in
// [4, 64] that still yields >= 1024 workgroups (4 per CU on 256 CUs).
inline int sweep_strip_rows(int B, int M) {
    int r = 64;
    while (r > 4 && int64_t(B) * ((M + r - 1) / r) < 1024) r /= 2;
    return r;
}

// dot_sinkhorn_forward with an optional per-iteration K scale (a tau
// schedule): ks_host[t] on the host and ks_dev[t] on the device for
// t < max_iter, or both null.  Defined in sinkhorn.hip.
int sinkhorn_forward_scheduled(const dot_sinkhorn_fwd_args* a, const float* ks_host, const float* ks_dev,
                               hipStream_t stream);

// Bytes of the forward's workspace without the persistent tier's optional
// scaled kernel (what dot_sinkhorn_forward needs at the least); 0 for a
// negative size.  Defined in sinkhorn.hip.
size_t forward_workspace_base_bytes(int B, int M, int N, int max_iter);

// sweep_strip_rows, or the value of DOT_AMD_ROWS when set (tuning only).
inline int tuned_strip_rows(int B, int M) {
    static const int forced = [] {
        const char* s = std::getenv("DOT_AMD_ROWS");
        return s ? std::atoi(s) : 0;
    }();
    return forced >= 1 ? forced : sweep_strip_rows(B, M);
}

}  // namespace dot_amd
