// Error reporting, version and the optional event profiler of the C ABI.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "host.hpp"

namespace dot_amd {
namespace {

thread_local std::string g_last_error;

struct Pending {
    const char* name;
    hipEvent_t start;
    hipEvent_t stop;
};

struct Total {
    int64_t launches = 0;
    double ms = 0.0;
};

struct Profiler {
    std::mutex mu;
    bool enabled = false;
    std::string select;  // ",name1,name2," or empty for every kernel
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
    std::map<std::string, Total> totals;
};

Profiler& profiler() {
    static Profiler* p = new Profiler();  // never destroyed: events may outlive static teardown
    return *p;
}

}  // namespace

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int ok() {
    g_last_error.clear();
    return DOT_OK;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(DOT_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return ok();
}

bool profiling_enabled(const char* name) {
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    if (!p.enabled) return false;
    if (p.select.empty()) return true;
    return p.select.find("," + std::string(name) + ",") != std::string::npos;
}

hipEvent_t profile_event() {
    Profiler& p = profiler();
    {
        std::lock_guard<std::mutex> lock(p.mu);
        if (!p.pool.empty()) {
            hipEvent_t e = p.pool.back();
            p.pool.pop_back();
            return e;
        }
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void profile_push(const char* name, hipEvent_t start, hipEvent_t stop) {
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    p.pending.push_back({name, start, stop});
}

}  // namespace dot_amd

using namespace dot_amd;

extern "C" const char* dot_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* dot_version(void) { return "dot_amd 0.1.0 (gfx950)"; }

extern "C" void dot_profile_enable(int on) {
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    p.enabled = on != 0;
}

extern "C" void dot_profile_select(const char* names) {
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    p.select = (names && *names) ? "," + std::string(names) + "," : std::string();
}

extern "C" int dot_profile_collect(void) {
    Profiler& p = profiler();
    std::vector<Pending> work;
    {
        std::lock_guard<std::mutex> lock(p.mu);
        work.swap(p.pending);
    }
    int rc = DOT_OK;
    for (const Pending& w : work) {
        float ms = 0.0f;
        if (hipEventSynchronize(w.stop) != hipSuccess ||
            hipEventElapsedTime(&ms, w.start, w.stop) != hipSuccess) {
            rc = fail(DOT_ERR_HIP, std::string("profiler: event wait failed for ") + w.name);
            continue;
        }
        std::lock_guard<std::mutex> lock(p.mu);
        Total& t = p.totals[w.name];
        t.launches += 1;
        t.ms += ms;
        p.pool.push_back(w.start);
        p.pool.push_back(w.stop);
    }
    return rc == DOT_OK ? ok() : rc;
}

extern "C" int dot_profile_query(const char* kernel, int64_t* launches, double* total_ms) {
    if (!kernel || !launches || !total_ms) return fail(DOT_ERR_INVALID_ARG, "NULL argument");
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    auto it = p.totals.find(kernel);
    *launches = it == p.totals.end() ? 0 : it->second.launches;
    *total_ms = it == p.totals.end() ? 0.0 : it->second.ms;
    return ok();
}

extern "C" void dot_profile_reset(void) {
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    p.totals.clear();
}

// Events still alive when the process exits are torn down after the HIP
// runtime (and any profiling tool attached to it) has shut down; a process
// that had created them then faulted inside exit().  This destroys every event
// the profiler owns while the runtime is still up.
extern "C" int dot_profile_shutdown(void) {
    Profiler& p = profiler();
    std::vector<Pending> work;
    std::vector<hipEvent_t> pool;
    {
        std::lock_guard<std::mutex> lock(p.mu);
        p.enabled = false;
        work.swap(p.pending);
        pool.swap(p.pool);
    }
    int rc = DOT_OK;
    for (const Pending& w : work) {
        if (hipEventSynchronize(w.stop) != hipSuccess)
            rc = fail(DOT_ERR_HIP, std::string("profiler: event wait failed for ") + w.name);
        pool.push_back(w.start);
        pool.push_back(w.stop);
    }
    for (hipEvent_t e : pool)
        if (hipEventDestroy(e) != hipSuccess) rc = fail(DOT_ERR_HIP, "profiler: hipEventDestroy failed");
    return rc == DOT_OK ? ok() : rc;
}
