// Sinkhorn C ABI: argument checks, workspace layout and the launch sequences.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "coop.hpp"
#include "host.hpp"
#include "persistent.cuh"
#include "resident.cuh"
#include "sinkhorn_kernels.cuh"
#include "wide.cuh"

namespace dot_amd {
namespace {

using sk::kColSumFloor;

int strip_rows(int B, int M) { return tuned_strip_rows(B, M); }

size_t lds_bytes(int N) { return (size_t(2) * N + 8) * sizeof(float); }


// Upper bound on the workgroups of a resident launch: at most kMaxGroup per
// batch element, at least 16 rows each, and at most 1024 in all.
size_t resident_groups_max(int B, int M, int N) {
    if (N > 1024 || N < 1) return 0;
    const size_t per_b = size_t(std::min((M + res::kWaves - 1) / res::kWaves, res::kMaxGroup));
    return std::min<size_t>(size_t(B) * per_b, 1024);
}

// Upper bound on the workgroups of a persistent streaming launch (at most
// pst::kMaxGroups per batch element, at most 1024 in all).
size_t pst_groups_max(int B, int M, int N) {
    if (N > kMaxRowLen || N < 1 || M < 1) return 0;
    return std::min<size_t>(size_t(B) * size_t(std::min(M, pst::kMaxGroups)), 1024);
}

struct FwdLayout {
    uint32_t* delta;
    float* ubuf;
    float* vbuf;
    size_t zero_words;
    float* partial;
    float2* rpart;              // rows longer than kMaxRowLen: [B, nchunks, M] row partials
    float* cost_partial;
    // resident path: tagged exchange slots, cleared before each resident launch
    unsigned long long* xchg;   // [2, G, N]
    unsigned long long* fxchg;  // [2, 2, G, N]
    unsigned long long* dxchg;  // [kDeltaSlots, G], then [G] cost partials
    int* status;
    size_t groups;
    size_t res_words;           // 32-bit words from xchg through status
    unsigned long long* pst;    // persistent streaming path: tagged slots, laid out per launch
    size_t pst_groups;
    int rows, nstrips, nchunks;
    size_t bytes;
};

// Column chunks of a row in the streaming sweeps: 1 when the row fits a
// wave's registers, else rows are swept in wide::kChunk-column tiles.
int row_chunks(int N) { return N > kMaxRowLen ? wide::num_chunks(N) : 1; }

int sweep_rows(int B, int M, int nchunks) {
    return nchunks > 1 ? wide::strip_rows(B, M, nchunks) : strip_rows(B, M);
}

FwdLayout fwd_layout(void* ws, int B, int M, int N, int max_iter) {
    Carver c(ws);
    FwdLayout L{};
    L.delta = c.take<uint32_t>(size_t(max_iter) + 1);
    L.ubuf = c.take<float>(size_t(2) * B * M);
    L.vbuf = c.take<float>(size_t(2) * B * N);
    L.zero_words = c.used() / sizeof(uint32_t);
    L.nchunks = row_chunks(N);
    L.rows = sweep_rows(B, M, L.nchunks);
    L.nstrips = (M + L.rows - 1) / L.rows;
    L.partial = c.take<float>(size_t(B) * L.nstrips * N);
    L.rpart = c.take<float2>(L.nchunks > 1 ? size_t(B) * L.nchunks * M : 0);
    L.pst_groups = pst_groups_max(B, M, N);
    L.cost_partial = c.take<float>(
        std::max(size_t(B) * std::max(size_t(L.nstrips) * L.nchunks, size_t(res::kMaxGroup)), L.pst_groups));
    L.groups = resident_groups_max(B, M, N);
    const size_t gn = L.groups * size_t(N);
    const size_t words = 6 * gn + (res::kDeltaSlots + 1) * L.groups + 1;
    L.xchg = c.take<unsigned long long>(words);
    if (L.xchg) {
        L.fxchg = L.xchg + 2 * gn;
        L.dxchg = L.fxchg + 4 * gn;
        L.status = reinterpret_cast<int*>(L.dxchg + (res::kDeltaSlots + 1) * L.groups);
    }
    L.res_words = 2 * words;
    // [2, G, N] partial rows | [2, B, N] v | [2, B, M] u | deltas [kDeltaSlots, G] | status
    L.pst = c.take<unsigned long long>(L.pst_groups ? 2 * L.pst_groups * size_t(N) + 2 * size_t(B) * N +
                                                          2 * size_t(B) * M + res::kDeltaSlots * L.pst_groups + 1
                                                    : 0);
    L.bytes = c.used();
    return L;
}

struct ImpLayout {
    float *r, *rs, *lam, *c, *cs, *mu, *partA, *partB, *tau_partial;
    float2* rpart;             // rows longer than kMaxRowLen: [B, nchunks, M] prologue row partials
    float* dpart;              // ... and [B, nchunks, M] row partials of each sweep
    unsigned long long* xchg;  // resident path: tagged exchange slots, then status
    int* status;
    size_t groups;             // workgroups the slots are laid out for
    size_t xchg_words;         // 32-bit words to clear (slots and status)
    unsigned long long* pst;   // persistent streaming path: tagged slots, laid out per launch
    size_t pst_groups;
    int rows, nstrips, nchunks;
    size_t bytes;
};

ImpLayout imp_layout(void* ws, int B, int M, int N) {
    Carver c(ws);
    ImpLayout L{};
    L.nchunks = row_chunks(N);
    L.rows = sweep_rows(B, M, L.nchunks);
    L.nstrips = (M + L.rows - 1) / L.rows;
    L.r = c.take<float>(size_t(B) * M);
    L.rs = c.take<float>(size_t(B) * M);
    L.lam = c.take<float>(size_t(B) * M);
    L.c = c.take<float>(size_t(B) * N);
    L.cs = c.take<float>(size_t(B) * N);
    L.mu = c.take<float>(size_t(B) * N);
    L.partA = c.take<float>(size_t(B) * L.nstrips * N);
    L.partB = c.take<float>(size_t(B) * L.nstrips * N);
    L.tau_partial = c.take<float>(size_t(B) * std::max(size_t(L.nstrips) * L.nchunks, size_t(pst::kMaxGroups)));
    L.rpart = c.take<float2>(L.nchunks > 1 ? size_t(B) * L.nchunks * M : 0);
    L.dpart = c.take<float>(L.nchunks > 1 ? size_t(B) * L.nchunks * M : 0);
    // The resident path runs at most one workgroup per CU and only for N <= 1024.
    const size_t groups = resident_groups_max(B, M, N);
    // [2, G, N] sweep slots, [2, G, N] prologue slots, [2, G] result words, then the status word
    L.groups = groups;
    const size_t words = 4 * groups * size_t(N) + 2 * groups + 1;
    L.xchg = c.take<unsigned long long>(words);
    L.status = reinterpret_cast<int*>(L.xchg ? L.xchg + words - 1 : nullptr);
    L.xchg_words = words * 2;
    // [2, G, N] sweep rows | [2, B, N + kMaxGroups] mu and stop-test scales | [2, G, N] prologue rows | status
    L.pst_groups = pst_groups_max(B, M, N);
    L.pst = c.take<unsigned long long>(
        L.pst_groups ? 4 * L.pst_groups * size_t(N) + 2 * size_t(B) * (size_t(N) + pst::kMaxGroups) + 1 : 0);
    L.bytes = c.used();
    return L;
}

struct UnrLayout {
    float *gamma, *partial, *colsum, *tau_partial;
    float* tpart;  // rows longer than kMaxRowLen: [B, nchunks, M] row partials of each step
    unsigned long long* pst;  // persistent streaming path: [2, G, N] rows | [2, B, N] sums | status
    size_t pst_groups;
    int rows, nstrips, nchunks;
    size_t bytes;
};

UnrLayout unr_layout(void* ws, int B, int M, int N) {
    Carver c(ws);
    UnrLayout L{};
    L.nchunks = row_chunks(N);
    L.rows = sweep_rows(B, M, L.nchunks);
    L.nstrips = (M + L.rows - 1) / L.rows;
    L.gamma = c.take<float>(size_t(B) * M * N);
    L.partial = c.take<float>(size_t(B) * L.nstrips * N);
    L.colsum = c.take<float>(size_t(B) * N);
    L.pst_groups = pst_groups_max(B, M, N);
    L.tau_partial = c.take<float>(std::max(size_t(B) * L.nstrips * L.nchunks, L.pst_groups));
    L.tpart = c.take<float>(L.nchunks > 1 ? size_t(B) * L.nchunks * M : 0);
    L.pst = c.take<unsigned long long>(L.pst_groups ? 2 * L.pst_groups * size_t(N) + 2 * size_t(B) * N + 1 : 0);
    L.bytes = c.used();
    return L;
}

__global__ void set_counts(int32_t* iters_used, int32_t* converged, int used, int conv) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *iters_used = used;
        *converged = conv;
    }
}

__global__ void set_status(int32_t* status, int value) {
    if (blockIdx.x == 0 && threadIdx.x == 0) *status = value;
}

__global__ void fill_value(float* p, size_t n, float value) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += size_t(gridDim.x) * blockDim.x)
        p[i] = value;
}

void launch_fill_zero(void* p, size_t words, hipStream_t stream) {
    if (words == 0) return;
    ProfScope prof("dot_fill_zero", stream);
    if (reinterpret_cast<uintptr_t>(p) % 16 == 0) {
        const unsigned blocks = unsigned(std::min<size_t>((words / 4 + kBlock - 1) / kBlock + 1, 2048));
        hipLaunchKernelGGL(sk::fill_zero16, dim3(blocks), dim3(kBlock), 0, stream, static_cast<uint32_t*>(p),
                           words);
        return;
    }
    const unsigned blocks = unsigned(std::min<size_t>((words + kBlock - 1) / kBlock, 2048));
    hipLaunchKernelGGL(sk::fill_zero, dim3(blocks), dim3(kBlock), 0, stream,
                       static_cast<uint32_t*>(p), words);
}

// Caller-owned exchange words of the register-resident kernels (the
// `exchange` fields): word 0 is the status, whose failure mark is the call's
// epoch; the tagged slots follow at kExchangeHead, tagged (epoch << 16) | t.
// The slots of the forward ([2, G, N] column sums, [2, 2, G, N] exact-LSE
// rows, [kDeltaSlots, G] deltas, [G] cost partials) are the larger set; the
// adjoint's ([2, G, N] sweep sums, [2, G, N] prologue sums, [2, G] result
// words) fit in them.  The result words of either launch are tagged
// (epoch << 16) | 0xfffe.
constexpr size_t kExchangeHead = 32;  // 256 bytes

size_t exchange_groups_max() { return size_t(std::max(0, std::min(device_cus(), 1024))); }

struct Tagging {
    unsigned long long* slots;
    int* status;
    unsigned tag_base, xcc_tag, result_tag;
    int mark;
    bool cleared_per_call;  // slots from the workspace: clear them before the launch
};

Tagging tagging(void* exchange, uint32_t epoch, int iters, unsigned long long* ws_slots, int* ws_status) {
    if (exchange && iters <= DOT_SINKHORN_MAX_TAGGED_ITERS) {
        const unsigned base = epoch << 16;
        return {static_cast<unsigned long long*>(exchange) + kExchangeHead, static_cast<int*>(exchange), base,
                base | 0xffffu, base | 0xfffeu, int(epoch), false};
    }
    return {ws_slots, ws_status, 0u, res::kXccTag, res::kResultTag, 1, true};
}

int check_exchange(const void* exchange, uint32_t epoch) {
    if (exchange && (epoch == 0 || epoch > DOT_SINKHORN_MAX_EPOCH))
        return fail(DOT_ERR_INVALID_ARG, "exchange_epoch must be in 1..DOT_SINKHORN_MAX_EPOCH");
    return DOT_OK;
}

int check_shape(int B, int M, int N) {
    if (B < 0 || M < 0 || N < 0) return fail(DOT_ERR_INVALID_ARG, "B, M and N must be >= 0");
    return DOT_OK;
}

bool valid_tau(float tau) { return std::isfinite(tau) && tau > 0.0f; }

// Register-resident configuration: a batch element's rows split over W
// workgroups of 8 waves, each wave holding RPW rows of PL floats per lane in
// VGPRs (PL * RPW <= strip_budget), one workgroup per CU.
struct ResidentCfg {
    bool ok = false;
    int vec = 1, ch = 1, rpw = 1, W = 1, R = 1;
};

// Resident strip budget (floats per lane) for a kernel and row width PL: the
// forward needs more working registers per row than the adjoint, so with
// 16-float rows it keeps 64 floats of strip instead of 128.
template <bool Forward>
constexpr int strip_budget(int pl) {
    return (Forward && pl >= 16) ? res::kMaxRegFloats / 2 : res::kMaxRegFloats;
}

template <bool Forward>
ResidentCfg resident_config(int B, int M, int N, bool vec4) {
    ResidentCfg c;
    const char* env = std::getenv("DOT_AMD_RESIDENT");
    if (env && env[0] == '0') return c;
    if (N < 1 || N > 1024 || M < 1 || B < 1) return c;
    if (N <= 64) {
        c.vec = 1;
        c.ch = 1;
    } else if (vec4) {
        c.vec = 4;
        c.ch = pow2_ceil((N + 255) / 256);
    } else {
        c.vec = 1;
        c.ch = pow2_ceil((N + 63) / 64);
    }
    const int pl = c.vec * c.ch;
    int rpw_max = 16;
    while (rpw_max > 1 && pl * rpw_max > strip_budget<Forward>(pl)) rpw_max /= 2;
    const int per_wg = res::kWaves * rpw_max;
    c.W = (M + per_wg - 1) / per_wg;
    if (c.W > res::kMaxGroup) return c;
    const int cus = device_cus();
    if (cus <= 0 || int64_t(B) * c.W > std::min(cus, 1024)) return c;
    c.R = (M + c.W - 1) / c.W;
    c.rpw = pow2_ceil((c.R + res::kWaves - 1) / res::kWaves);
    c.ok = c.rpw <= rpw_max;
    return c;
}

template <bool Forward, class F>
bool dispatch_resident(const ResidentCfg& c, F&& f) {
    constexpr bool Fwd = Forward;
    using std::integral_constant;
    auto rows = [&](auto vc, auto cc) {
        constexpr int PL = decltype(vc)::value * decltype(cc)::value;
        switch (c.rpw) {
            case 1: f(vc, cc, integral_constant<int, 1>{}); return true;
            case 2: if constexpr (PL * 2 <= strip_budget<Fwd>(PL)) { f(vc, cc, integral_constant<int, 2>{}); return true; } break;
            case 4: if constexpr (PL * 4 <= strip_budget<Fwd>(PL)) { f(vc, cc, integral_constant<int, 4>{}); return true; } break;
            case 8: if constexpr (PL * 8 <= strip_budget<Fwd>(PL)) { f(vc, cc, integral_constant<int, 8>{}); return true; } break;
            case 16: if constexpr (PL * 16 <= strip_budget<Fwd>(PL)) { f(vc, cc, integral_constant<int, 16>{}); return true; } break;
        }
        return false;
    };
    if (c.vec == 4) {
        switch (c.ch) {
            case 1: return rows(integral_constant<int, 4>{}, integral_constant<int, 1>{});
            case 2: return rows(integral_constant<int, 4>{}, integral_constant<int, 2>{});
            case 4: return rows(integral_constant<int, 4>{}, integral_constant<int, 4>{});
        }
        return false;
    }
    switch (c.ch) {
        case 1: return rows(integral_constant<int, 1>{}, integral_constant<int, 1>{});
        case 2: return rows(integral_constant<int, 1>{}, integral_constant<int, 2>{});
        case 4: return rows(integral_constant<int, 1>{}, integral_constant<int, 4>{});
        case 8: return rows(integral_constant<int, 1>{}, integral_constant<int, 8>{});
        case 16: return rows(integral_constant<int, 1>{}, integral_constant<int, 16>{});
    }
    return false;
}

// Persistent streaming configuration: W workgroups per batch element (as many
// as the CUs allow, at most pst::kMaxGroups and M), R rows each.
struct StreamCfg {
    bool ok = false;
    int W = 1, R = 1;
};

StreamCfg stream_config(int B, int M, int N) {
    StreamCfg c;
    const char* env = std::getenv("DOT_AMD_PERSISTENT");
    if (env && env[0] == '0') return c;
    if (N < 1 || N > kMaxRowLen || M < 1 || B < 1) return c;
    const int cus = device_cus();
    if (cus <= 0 || B > cus) return c;
    c.W = std::min({cus / B, pst::kMaxGroups, M});
    if (int64_t(B) * c.W > 1024) return c;
    c.R = (M + c.W - 1) / c.W;
    c.ok = true;
    return c;
}

// Bytes of the persistent forward's scaled kernel E (pst::forward, scaling
// domain) for shapes that take that tier; the workspace query includes them,
// and a smaller workspace that still holds fwd_layout runs without E.
size_t scaled_kernel_bytes(int B, int M, int N) {
    // rows of 64 floats per lane only (pst::forward)
    if (N <= 2048 || resident_config<true>(B, M, N, N % 4 == 0).ok || !stream_config(B, M, N).ok) return 0;
    return (size_t(B) * M * N * sizeof(float) + 255) & ~size_t(255);
}

float* scaled_kernel(const dot_sinkhorn_fwd_args* a, const FwdLayout& L) {
    const size_t ek = scaled_kernel_bytes(a->B, a->M, a->N);
    if (ek == 0 || !a->workspace || a->workspace_bytes < L.bytes + ek) return nullptr;
    return reinterpret_cast<float*>(static_cast<char*>(a->workspace) + L.bytes);
}

bool launch_stream_forward(const dot_sinkhorn_fwd_args* a, const FwdLayout& L, const StreamCfg& sc,
                           float kscale, const float* ks_dev, float log_a_default, float log_b_default,
                           bool keep, bool ret_log, bool vec4, float* ebuf, hipStream_t stream) {
    const int B = a->B, M = a->M, N = a->N, G = B * sc.W;
    if (!L.pst || size_t(G) > L.pst_groups) return false;
    pst::FwdArgs r{};
    r.X = a->scores;
    r.kscale = kscale;
    r.kscale_t = ks_dev;
    r.scores_kind = a->scores_kind;
    r.log_a = a->log_a;
    r.log_b = a->log_b;
    r.log_a_default = log_a_default;
    r.log_b_default = log_b_default;
    r.tol = a->tol;
    r.max_iter = a->max_iter;
    r.return_log = ret_log ? 1 : 0;
    r.plan = a->plan;
    r.cost_partial = a->cost ? L.cost_partial : nullptr;
    r.u_out = a->u_out;
    r.v_out = a->v_out;
    r.u_hist = keep ? a->u_hist : nullptr;
    r.v_hist = keep ? a->v_hist : nullptr;
    r.iters_used = a->iters_used;
    r.converged = a->converged;
    r.part = L.pst;
    r.res = r.part + 2 * size_t(G) * N;
    r.uslot = r.res + 2 * size_t(B) * N;
    r.dxchg = r.uslot + 2 * size_t(B) * M;
    r.status = reinterpret_cast<int*>(r.dxchg + res::kDeltaSlots * size_t(G));
    r.B = B;
    r.M = M;
    r.N = N;
    r.W = sc.W;
    r.R = sc.R;
    r.spin_limit = spin_limit();
    r.local_ok = local_exchange_allowed();
    r.ebuf = ks_dev ? nullptr : ebuf;
    const size_t words = size_t(reinterpret_cast<unsigned long long*>(r.status) - L.pst) + 1;
    bool ok = false;
    dispatch_row(N, vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        // fold rows | v, v log2(e), log b | red (padded to 4) | u 2R, log a R, row maxima R | scratch
        const size_t lds = (size_t(pst::kFoldRows<V, C> + 3) * N + ((size_t(N) + sc.W + 3) & ~size_t(3)) +
                            4 * size_t(sc.R) + res::kFwdScratch) *
                           sizeof(float);
        launch_fill_zero(L.pst, 2 * words, stream);
        ProfScope prof("sk_fwd_persistent", stream);
        ok = ks_dev ? launch_persistent(pst::forward<V, C, true>, r, G, res::kThreads, lds, stream)
                    : launch_persistent(pst::forward<V, C>, r, G, res::kThreads, lds, stream);
    });
    if (!ok) return false;
    if (a->cost) {
        ProfScope prof("sk_batch_sum", stream);
        hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.cost_partial, sc.W, 1.0f,
                           a->cost);
    }
    return true;
}

// Launch of the register-resident forward; false when this shape or
// device cannot host it (the caller then runs the streaming sweeps).
bool launch_resident_forward(const dot_sinkhorn_fwd_args* a, const FwdLayout& L, const ResidentCfg& rc,
                             float kscale, const float* ks_dev, float log_a_default, float log_b_default,
                             bool keep, bool ret_log, hipStream_t stream) {
    const int groups = a->B * rc.W;
    if (!L.xchg || size_t(groups) > L.groups) return false;
    res::FwdResArgs r{};
    r.X = a->scores;
    r.kscale = kscale;
    r.kscale_t = ks_dev;
    r.scores_kind = a->scores_kind;
    r.log_a = a->log_a;
    r.log_b = a->log_b;
    r.log_a_default = log_a_default;
    r.log_b_default = log_b_default;
    r.tol = a->tol;
    r.max_iter = a->max_iter;
    r.return_log = ret_log ? 1 : 0;
    r.plan = a->plan;
    r.cost = a->cost;
    r.u_out = a->u_out;
    r.v_out = a->v_out;
    r.u_hist = keep ? a->u_hist : nullptr;
    r.v_hist = keep ? a->v_hist : nullptr;
    r.iters_used = a->iters_used;
    r.converged = a->converged;
    // The exchange regions are laid out for L.groups workgroups; index them by the real grid.
    const Tagging tg = tagging(a->exchange, a->exchange_epoch, a->max_iter, L.xchg, L.status);
    r.xchg = tg.slots;
    r.fxchg = tg.slots + 2 * size_t(groups) * a->N;
    r.dxchg = r.fxchg + 4 * size_t(groups) * a->N;
    r.cwords = r.dxchg + res::kDeltaSlots * size_t(groups);
    r.result_tag = tg.result_tag;
    r.status = tg.status;
    r.tag_base = tg.tag_base;
    r.xcc_tag = tg.xcc_tag;
    r.mark = tg.mark;
    r.B = a->B;
    r.M = a->M;
    r.N = a->N;
    r.W = rc.W;
    r.R = rc.R;
    r.spin_limit = spin_limit();
    r.local_ok = local_exchange_allowed();
    // DOT_AMD_EXACT_ROWMAX=1: every row update shifts by the row maximum
    const char* exact_max = std::getenv("DOT_AMD_EXACT_ROWMAX");
    r.lagged_shift = (exact_max && exact_max[0] == '1') ? 0 : 1;
    bool ok = false;
    dispatch_resident<true>(rc, [&](auto vc, auto cc, auto rr) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        constexpr int RPW = decltype(rr)::value;
        const size_t lds =
            (size_t(12) * a->N + 3 * res::kWaves * RPW + res::kFwdScratch) * sizeof(float);
        auto kernel = ks_dev ? res::forward<V, C, RPW, true> : res::forward<V, C, RPW>;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, res::kThreads, lds) != hipSuccess ||
            per_cu < 1 || int64_t(per_cu) * device_cus() < groups)
            return;
        if (tg.cleared_per_call) launch_fill_zero(L.xchg, L.res_words, stream);
        void* params[] = {&r};
        ProfScope prof("sk_fwd_resident", stream);
        // one workgroup per element exchanges only with itself; the stop test
        // (tol > 0) couples all workgroups of the batch
        const bool independent = rc.W == 1 && (!(a->tol > 0.0f) || groups == 1);
        ok = launch_grid(reinterpret_cast<const void*>(kernel), groups, res::kThreads, params, lds, stream,
                         independent) == hipSuccess;
    });
    return ok;
}

// The per-iteration forward sweeps with tol > 0 read the device's stop test
// back after iterations 4, 8, 16, ... (one wait on the stream each) and stop
// launching once it has fired: delta[t] < tol, where an iteration that did not
// run left 0.  The launches of a stopped run return at once, but each still
// costs ~2.5 us of the queue, which at C3's shape (stop at 5 of 200) was most
// of the step.  Not on a stream under capture: a replay could not re-decide.
struct StopCheck {
    const uint32_t* delta;
    float tol;
    bool on = false;
    int rc = DOT_OK;

    StopCheck(const uint32_t* d, float t, int max_iter, hipStream_t stream) : delta(d), tol(t) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        on = tol > 0.0f && max_iter > 4 && hipStreamIsCapturing(stream, &cs) == hipSuccess &&
             cs == hipStreamCaptureStatusNone;
    }

    // true when iteration t (1-based, just launched) ends the launches
    bool stopped(int t, int max_iter, hipStream_t stream) {
        if (!on || t < 4 || (t & (t - 1)) != 0 || t >= max_iter) return false;
        uint32_t w = 0;
        if (hipMemcpyAsync(&w, delta + t, sizeof(w), hipMemcpyDeviceToHost, stream) != hipSuccess ||
            hipStreamSynchronize(stream) != hipSuccess) {
            rc = fail(DOT_ERR_HIP, "dot_sinkhorn_forward: stop-flag read failed");
            return true;
        }
        float d;
        std::memcpy(&d, &w, sizeof(d));
        return d < tol;
    }
};

// Rows longer than kMaxRowLen: per iteration a rows pass (chunk partials of
// the row log-sum-exp), a columns pass (u and the column sums) and the column
// combine; then the plan in chunk tiles.  The workspace's delta and potential
// buffers are already cleared.
int launch_wide_forward(const dot_sinkhorn_fwd_args* a, const FwdLayout& L, const float* ks_host,
                        float kscale, float log_a_default, float log_b_default, bool keep, bool ret_log,
                        bool vec4, hipStream_t stream) {
    const int B = a->B, M = a->M, N = a->N, T = a->max_iter;
    StopCheck stop(L.delta, a->tol, T, stream);
    const dim3 tiles = batch_grid(unsigned(L.nstrips) * unsigned(L.nchunks), B);
    const size_t lds = (size_t(2) * wide::kChunk + 8) * sizeof(float);
    wide::dispatch_chunk(vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        for (int t = 1; t <= T; ++t) {
            const int cur = t & 1, prev = (t - 1) & 1;
            const float ks = ks_host ? ks_host[t - 1] : kscale;
            wide::FwdArgs w{};
            w.X = a->scores;
            w.kscale = ks;
            w.log_a = a->log_a;
            w.log_a_default = log_a_default;
            w.v_old = L.vbuf + size_t(prev) * B * N;
            w.u_old = L.ubuf + size_t(prev) * B * M;
            w.u_new = L.ubuf + size_t(cur) * B * M;
            w.u_hist = keep ? a->u_hist + size_t(t - 1) * B * M : nullptr;
            w.rpart = L.rpart;
            w.partial = L.partial;
            w.delta_bits = L.delta;
            w.B = B;
            w.M = M;
            w.N = N;
            w.rows = L.rows;
            w.nstrips = L.nstrips;
            w.nchunks = L.nchunks;
            w.t = t;
            w.tol = a->tol;
            {
                ProfScope prof("sk_fwd_wide_rows", stream);
                hipLaunchKernelGGL((wide::fwd_rows<V, C>), tiles, dim3(kBlock), 0, stream, w);
            }
            {
                ProfScope prof("sk_fwd_wide_cols", stream);
                hipLaunchKernelGGL((wide::fwd_cols<V, C>), tiles, dim3(kBlock), lds, stream, w);
            }
            sk::FwdCombineArgs cb{};
            cb.partial = L.partial;
            cb.nstrips = L.nstrips;
            cb.X = a->scores;
            cb.kscale = ks;
            cb.u_new = w.u_new;
            cb.log_b = a->log_b;
            cb.log_b_default = log_b_default;
            cb.v_old = w.v_old;
            cb.v_new = L.vbuf + size_t(cur) * B * N;
            cb.v_hist = keep ? a->v_hist + size_t(t - 1) * B * N : nullptr;
            cb.delta_bits = L.delta;
            cb.tol = a->tol;
            cb.t = t;
            cb.B = B;
            cb.M = M;
            cb.N = N;
            {
                ProfScope prof("sk_fwd_combine", stream);
                hipLaunchKernelGGL(sk::fwd_combine, sk::fold_grid(N, B), dim3(kBlock), 0, stream, cb);
            }
            if (stop.stopped(t, T, stream)) break;
        }
        {
            ProfScope prof("sk_fwd_finalize", stream);
            hipLaunchKernelGGL(sk::fwd_finalize, dim3(1), dim3(kWave), 0, stream, L.delta, T, a->tol,
                               a->iters_used, a->converged);
        }
        if (a->plan || a->cost || a->u_out || a->v_out) {
            sk::MaterializeArgs m{};
            m.X = a->scores;
            m.kscale = kscale;
            m.scores_kind = a->scores_kind;
            m.ubuf = L.ubuf;
            m.vbuf = L.vbuf;
            m.iters_used = a->iters_used;
            m.plan = a->plan;
            m.return_log = ret_log ? 1 : 0;
            m.cost_partial = a->cost ? L.cost_partial : nullptr;
            m.u_out = a->u_out;
            m.v_out = a->v_out;
            m.B = B;
            m.M = M;
            m.N = N;
            m.rows = L.rows;
            {
                ProfScope prof("sk_materialize", stream);
                hipLaunchKernelGGL((wide::materialize<V, C>), tiles, dim3(kBlock), 0, stream, m, L.nchunks);
            }
            if (a->cost) {
                ProfScope prof("sk_batch_sum", stream);
                hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.cost_partial,
                                   int(tiles.x), 1.0f, a->cost);
            }
        }
    });
    return stop.rc;
}

}  // namespace
}  // namespace dot_amd

using namespace dot_amd;

extern "C" size_t dot_sinkhorn_forward_workspace_bytes(int B, int M, int N, int max_iter, int flags) {
    (void)flags;
    if (B < 0 || M < 0 || N < 0 || max_iter < 0) return 0;
    return fwd_layout(nullptr, B, M, N, max_iter).bytes + scaled_kernel_bytes(B, M, N);
}

extern "C" size_t dot_sinkhorn_exchange_bytes(void) {
    const size_t G = exchange_groups_max();
    return (kExchangeHead + 6 * G * 1024 + (res::kDeltaSlots + 1) * G) * sizeof(unsigned long long);
}

extern "C" int dot_sinkhorn_forward(const dot_sinkhorn_fwd_args* a, dot_stream_t stream_) {
    return dot_amd::sinkhorn_forward_scheduled(a, nullptr, nullptr, reinterpret_cast<hipStream_t>(stream_));
}

// The forward with an optional per-iteration K scale (a tau schedule):
// ks_host[t] and its device copy ks_dev[t] for t < max_iter, or both null.
int dot_amd::sinkhorn_forward_scheduled(const dot_sinkhorn_fwd_args* a, const float* ks_host,
                                        const float* ks_dev, hipStream_t stream) {
    if (!a) return fail(DOT_ERR_INVALID_ARG, "args is NULL");
    if (int rc = check_shape(a->B, a->M, a->N)) return rc;
    if (!valid_tau(a->tau)) return fail(DOT_ERR_INVALID_ARG, "tau must be > 0");
    if (a->max_iter < 0) return fail(DOT_ERR_INVALID_ARG, "max_iter must be >= 0");
    if (a->scores_kind != DOT_SCORES_LOG_ALPHA && a->scores_kind != DOT_SCORES_COST)
        return fail(DOT_ERR_INVALID_ARG, "scores_kind must be DOT_SCORES_LOG_ALPHA or DOT_SCORES_COST");
    if (!a->iters_used || !a->converged)
        return fail(DOT_ERR_INVALID_ARG, "iters_used and converged must be device pointers");
    if (int rc = check_exchange(a->exchange, a->exchange_epoch)) return rc;
    const bool keep = (a->flags & DOT_SK_KEEP_HISTORY) != 0;
    const bool ret_log = (a->flags & DOT_SK_RETURN_LOG) != 0;
    if (a->flags & ~(DOT_SK_KEEP_HISTORY | DOT_SK_RETURN_LOG))
        return fail(DOT_ERR_INVALID_ARG, "unknown flag bits");
    if (ret_log && a->cost) return fail(DOT_ERR_INVALID_ARG, "cost is undefined with DOT_SK_RETURN_LOG");
    if (keep && a->max_iter > 0 && (!a->u_hist || !a->v_hist))
        return fail(DOT_ERR_INVALID_ARG, "DOT_SK_KEEP_HISTORY needs u_hist and v_hist");
    const int B = a->B, M = a->M, N = a->N, T = a->max_iter;
    const size_t elems = size_t(B) * M * N;

    if (elems == 0) {
        // Degenerate shapes: the reference's loop still runs one delta check of an
        // empty vector (delta = 0), so a positive tol reports convergence at t = 1.
        const bool stop = a->tol > 0.0f && T > 0;
        hipLaunchKernelGGL(set_counts, dim3(1), dim3(1), 0, stream, a->iters_used, a->converged,
                           stop ? 1 : T, stop ? 1 : 0);
        if (a->cost && B > 0) hipLaunchKernelGGL(fill_value, dim3(1), dim3(kBlock), 0, stream, a->cost, size_t(B), 0.0f);
        return check_launch("dot_sinkhorn_forward");
    }
    if (!a->scores) return fail(DOT_ERR_INVALID_ARG, "scores is NULL");

    const FwdLayout L = fwd_layout(a->workspace, B, M, N, T);
    if (!a->workspace || a->workspace_bytes < L.bytes)
        return fail(DOT_ERR_WORKSPACE, "workspace smaller than dot_sinkhorn_forward_workspace_bytes()");

    const float tau = a->tau;
    const float inv_tau = 1.0f / tau;                       // torch_cuda.cpp / kernels.cu:1350
    const float kscale = float(a->scores_kind) * inv_tau;
    const float log_a_default = -std::log(static_cast<float>(M));  // torch_cuda.cpp:42
    const float log_b_default = -std::log(static_cast<float>(N));
    const bool vec4 = (N % 4 == 0) && aligned16(a->scores) && (!a->plan || aligned16(a->plan));
    const size_t lds = lds_bytes(N);

    const ResidentCfg rc = resident_config<true>(B, M, N, vec4);
    if (rc.ok && launch_resident_forward(a, L, rc, kscale, ks_dev, log_a_default, log_b_default, keep, ret_log,
                                         stream))
        return check_launch("dot_sinkhorn_forward");
    (void)hipGetLastError();  // a refused cooperative launch falls back to the next tier
    const StreamCfg sc = stream_config(B, M, N);
    if (sc.ok && launch_stream_forward(a, L, sc, kscale, ks_dev, log_a_default, log_b_default, keep, ret_log,
                                       vec4, scaled_kernel(a, L), stream))
        return check_launch("dot_sinkhorn_forward");
    (void)hipGetLastError();

    launch_fill_zero(a->workspace, L.zero_words, stream);
    if (L.nchunks > 1) {
        if (int rc = launch_wide_forward(a, L, ks_host, kscale, log_a_default, log_b_default, keep, ret_log, vec4,
                                         stream))
            return rc;
        return check_launch("dot_sinkhorn_forward");
    }

    StopCheck stop(L.delta, a->tol, T, stream);
    bool launched = dispatch_row(N, vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        for (int t = 1; t <= T; ++t) {
            const int cur = t & 1, prev = (t - 1) & 1;
            const float ks = ks_host ? ks_host[t - 1] : kscale;
            sk::FwdSweepArgs s{};
            s.X = a->scores;
            s.kscale = ks;
            s.log_a = a->log_a;
            s.log_a_default = log_a_default;
            s.v_old = L.vbuf + size_t(prev) * B * N;
            s.u_old = L.ubuf + size_t(prev) * B * M;
            s.u_new = L.ubuf + size_t(cur) * B * M;
            s.u_hist = keep ? a->u_hist + size_t(t - 1) * B * M : nullptr;
            s.partial = L.partial;
            s.delta_bits = L.delta;
            s.B = B;
            s.M = M;
            s.N = N;
            s.rows = L.rows;
            s.nstrips = L.nstrips;
            s.t = t;
            s.tol = a->tol;
            {
                ProfScope prof("sk_fwd_sweep", stream);
                hipLaunchKernelGGL((sk::fwd_sweep<V, C>), batch_grid(unsigned(L.nstrips), B), dim3(kBlock), lds,
                                   stream, s);
            }
            sk::FwdCombineArgs cb{};
            cb.partial = L.partial;
            cb.nstrips = L.nstrips;
            cb.X = a->scores;
            cb.kscale = ks;
            cb.u_new = s.u_new;
            cb.log_b = a->log_b;
            cb.log_b_default = log_b_default;
            cb.v_old = s.v_old;
            cb.v_new = L.vbuf + size_t(cur) * B * N;
            cb.v_hist = keep ? a->v_hist + size_t(t - 1) * B * N : nullptr;
            cb.delta_bits = L.delta;
            cb.tol = a->tol;
            cb.t = t;
            cb.B = B;
            cb.M = M;
            cb.N = N;
            {
                ProfScope prof("sk_fwd_combine", stream);
                hipLaunchKernelGGL(sk::fwd_combine, sk::fold_grid(N, B), dim3(kBlock), 0, stream, cb);
            }
            if (stop.stopped(t, T, stream)) break;
        }
        {
            ProfScope prof("sk_fwd_finalize", stream);
            hipLaunchKernelGGL(sk::fwd_finalize, dim3(1), dim3(kWave), 0, stream, L.delta, T,
                               a->tol, a->iters_used, a->converged);
        }
        if (a->plan || a->cost || a->u_out || a->v_out) {
            sk::MaterializeArgs m{};
            m.X = a->scores;
            m.kscale = kscale;
            m.scores_kind = a->scores_kind;
            m.ubuf = L.ubuf;
            m.vbuf = L.vbuf;
            m.iters_used = a->iters_used;
            m.plan = a->plan;
            m.return_log = ret_log ? 1 : 0;
            m.cost_partial = a->cost ? L.cost_partial : nullptr;
            m.u_out = a->u_out;
            m.v_out = a->v_out;
            m.B = B;
            m.M = M;
            m.N = N;
            m.rows = L.rows;
            {
                ProfScope prof("sk_materialize", stream);
                hipLaunchKernelGGL((sk::materialize<V, C>), batch_grid(unsigned(L.nstrips), B), dim3(kBlock), 0,
                                   stream, m);
            }
            if (a->cost) {
                ProfScope prof("sk_batch_sum", stream);
                hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.cost_partial,
                                   L.nstrips, 1.0f, a->cost);
            }
        }
    });
    if (!launched) return fail(DOT_ERR_UNSUPPORTED, "row length outside the supported range");
    if (stop.rc) return stop.rc;
    return check_launch("dot_sinkhorn_forward");
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
namespace {

int check_bwd(const dot_sinkhorn_bwd_args* a) {
    if (!a) return fail(DOT_ERR_INVALID_ARG, "args is NULL");
    if (int rc = check_shape(a->B, a->M, a->N)) return rc;
    if (!valid_tau(a->tau)) return fail(DOT_ERR_INVALID_ARG, "tau must be > 0");
    if (a->iters < 0) return fail(DOT_ERR_INVALID_ARG, "iters must be >= 0");
    if (a->scores_kind != DOT_SCORES_LOG_ALPHA && a->scores_kind != DOT_SCORES_COST)
        return fail(DOT_ERR_INVALID_ARG, "scores_kind must be DOT_SCORES_LOG_ALPHA or DOT_SCORES_COST");
    const size_t elems = size_t(a->B) * a->M * a->N;
    if (elems > 0 && (!a->scores || !a->plan || !a->grad_scores))
        return fail(DOT_ERR_INVALID_ARG, "scores, plan and grad_scores must be non-NULL");
    if (a->B > 0 && !a->grad_tau) return fail(DOT_ERR_INVALID_ARG, "grad_tau must be non-NULL");
    if (a->flags & ~(DOT_SK_EXACT_SWEEPS | DOT_SK_GRAD_COST_SCALAR))
        return fail(DOT_ERR_INVALID_ARG, "unknown flag bits");
    return check_exchange(a->exchange, a->exchange_epoch);
}

__global__ void fill_int(int32_t* p, int n, int value) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = value;
}

// sweeps_used of a call whose adjoint runs every sweep.
void report_all_sweeps(const dot_sinkhorn_bwd_args* a, hipStream_t stream) {
    if (a->sweeps_used && a->B > 0)
        hipLaunchKernelGGL(fill_int, dim3(unsigned(std::min((a->B + kBlock - 1) / kBlock, 1024))), dim3(kBlock),
                           0, stream, a->sweeps_used, a->B, a->iters);
}

bool bwd_vec4(const dot_sinkhorn_bwd_args* a) {
    return (a->N % 4 == 0) && aligned16(a->scores) && aligned16(a->plan) &&
           aligned16(a->grad_scores) && (!a->grad_plan || aligned16(a->grad_plan));
}

sk::GradSource grad_source(const dot_sinkhorn_bwd_args* a) {
    sk::GradSource g{};
    g.X = a->scores;
    g.scores_kind = a->scores_kind;
    g.gP = a->grad_plan;
    g.gC = a->grad_cost;
    g.gc_step = (a->flags & DOT_SK_GRAD_COST_SCALAR) ? 0 : 1;
    return g;
}

// Zero gradients for empty matrices with a non-empty batch.
int bwd_degenerate(const dot_sinkhorn_bwd_args* a, hipStream_t stream, const char* what) {
    if (a->B > 0)
        hipLaunchKernelGGL(fill_value, dim3(1), dim3(kBlock), 0, stream, a->grad_tau, size_t(a->B), 0.0f);
    if (a->status) hipLaunchKernelGGL(set_status, dim3(1), dim3(1), 0, stream, a->status, 0);
    return check_launch(what);
}

}  // namespace

namespace {

// Launch of the register-resident adjoint; false when this shape or
// device cannot host it (the caller then runs the next tier).  keep_status:
// a later slab of the call (launch_resident_slabs), which must not clear the
// failure mark an earlier slab left in a->status.
bool launch_resident_adjoint(const dot_sinkhorn_bwd_args* a, const ImpLayout& L, const ResidentCfg& rc,
                             float inv_tau, hipStream_t stream, bool keep_status = false) {
    const int groups = a->B * rc.W;
    if (!L.xchg || size_t(groups) > L.groups) return false;
    res::ImpResArgs r{};
    r.X = a->scores;
    r.scores_kind = a->scores_kind;
    r.gP = a->grad_plan;
    r.gC = a->grad_cost;
    r.gc_step = (a->flags & DOT_SK_GRAD_COST_SCALAR) ? 0 : 1;
    r.P = a->plan;
    const Tagging tg = tagging(a->exchange, a->exchange_epoch, a->iters, L.xchg, L.status);
    r.xchg = tg.slots;
    r.pro = tg.slots + 2 * size_t(groups) * a->N;
    r.grad = a->grad_scores;
    r.grad_tau = a->grad_tau;
    r.tau_scale = -inv_tau;
    r.rwords = r.pro + 2 * size_t(groups) * a->N;
    r.result_tag = tg.result_tag;
    r.status_out = a->status;
    r.keep_status = keep_status ? 1 : 0;
    r.status = tg.status;
    r.tag_base = tg.tag_base;
    r.xcc_tag = tg.xcc_tag;
    r.mark = tg.mark;
    r.inv_tau = inv_tau;
    r.M = a->M;
    r.N = a->N;
    r.W = rc.W;
    r.R = rc.R;
    r.iters = a->iters;
    r.spin_limit = spin_limit();
    r.local_ok = local_exchange_allowed();
    r.sweeps = a->sweeps_used;
    r.early = (a->flags & DOT_SK_EXACT_SWEEPS) ? 0 : 1;
    bool ok = false;
    dispatch_resident<false>(rc, [&](auto vc, auto cc, auto rr) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        constexpr int RPW = decltype(rr)::value;
        // wave rows 8N | mu N | scratch 8 | the stop test's per-wave values 16
        const size_t lds = (size_t(res::kWaves + 1) * a->N + 3 * res::kWaves) * sizeof(float);
        // elements of at most 4 workgroups poll their exchange from fewer registers
        auto kernel = rc.W <= 4 ? res::implicit_adjoint<V, C, RPW, 4> : res::implicit_adjoint<V, C, RPW>;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, res::kThreads, lds) != hipSuccess ||
            per_cu < 1 || int64_t(per_cu) * device_cus() < groups)
            return;
        if (tg.cleared_per_call) launch_fill_zero(L.xchg, L.xchg_words, stream);
        void* params[] = {&r};
        ProfScope prof("sk_imp_resident", stream);
        // the adjoint's exchanges stay within a batch element's W workgroups,
        // but the status word waits for the whole grid
        ok = launch_grid(reinterpret_cast<const void*>(kernel), groups, res::kThreads, params, lds, stream,
                         rc.W == 1 && !a->status) == hipSuccess;
    });
    return ok;
}

// Elements per launch of the register-resident adjoint at this shape (the
// most that fit the chip's registers at once), or 0 when one does not fit.
int resident_slab(int B, int M, int N, bool vec4) {
    const ResidentCfg one = resident_config<false>(1, M, N, vec4);
    if (!one.ok) return 0;
    return std::min(B, std::max(1, std::min(device_cus(), 1024) / one.W));
}

// The arguments of batch elements [b0, b0 + n) of a backward call, with the
// exchange words left to the launch's own workspace (caller-owned words would
// repeat one epoch across the slabs).
dot_sinkhorn_bwd_args slab_args(const dot_sinkhorn_bwd_args* a, int b0, int n) {
    const size_t MN = size_t(a->M) * a->N;
    dot_sinkhorn_bwd_args s = *a;
    s.B = n;
    s.scores = a->scores + b0 * MN;
    s.plan = a->plan + b0 * MN;
    s.grad_plan = a->grad_plan ? a->grad_plan + b0 * MN : nullptr;
    s.grad_cost = a->grad_cost ? a->grad_cost + ((a->flags & DOT_SK_GRAD_COST_SCALAR) ? 0 : b0) : nullptr;
    s.grad_scores = a->grad_scores + b0 * MN;
    s.grad_tau = a->grad_tau + b0;
    s.sweeps_used = a->sweeps_used ? a->sweeps_used + b0 : nullptr;
    s.exchange = nullptr;
    s.exchange_epoch = 0;
    return s;
}

// A batch larger than a one-launch adjoint holds at once, in slabs of `slab`
// elements, one launch each on the stream: launch(slab arguments, whether an
// earlier slab ran).  The adjoint couples no batch elements, so every slab
// computes exactly its elements' share of the call, and each launch clears
// its own workspace exchange words.  False when a slab cannot be hosted; the
// caller then runs the whole batch on the next tier, which overwrites every
// output.
template <class Launch>
bool launch_slabs(const dot_sinkhorn_bwd_args* a, int slab, Launch&& launch) {
    for (int b0 = 0; b0 < a->B; b0 += slab) {
        const dot_sinkhorn_bwd_args s = slab_args(a, b0, std::min(slab, a->B - b0));
        if (!launch(s, b0 > 0)) return false;
    }
    return true;
}

bool launch_resident_slabs(const dot_sinkhorn_bwd_args* a, const ImpLayout& L, int slab, float inv_tau,
                           hipStream_t stream) {
    return launch_slabs(a, slab, [&](const dot_sinkhorn_bwd_args& s, bool keep) {
        const ResidentCfg rc = resident_config<false>(s.B, s.M, s.N, bwd_vec4(&s));
        return rc.ok && launch_resident_adjoint(&s, L, rc, inv_tau, stream, keep);
    });
}

bool launch_stream_adjoint(const dot_sinkhorn_bwd_args* a, const ImpLayout& L, const StreamCfg& sc,
                           float inv_tau, bool vec4, hipStream_t stream, bool keep_status = false) {
    const int B = a->B, N = a->N, G = B * sc.W;
    if (!L.pst || size_t(G) > L.pst_groups) return false;
    pst::ImpArgs r{};
    r.X = a->scores;
    r.scores_kind = a->scores_kind;
    r.gP = a->grad_plan;
    r.gC = a->grad_cost;
    r.gc_step = (a->flags & DOT_SK_GRAD_COST_SCALAR) ? 0 : 1;
    r.P = a->plan;
    r.part = L.pst;
    r.res = r.part + 2 * size_t(G) * N;
    r.pro = r.res + 2 * size_t(B) * (size_t(N) + pst::kMaxGroups);
    r.status = reinterpret_cast<int*>(r.pro + 2 * size_t(G) * N);
    r.grad = a->grad_scores;
    r.tau_partial = L.tau_partial;
    r.inv_tau = inv_tau;
    r.B = B;
    r.M = a->M;
    r.N = N;
    r.W = sc.W;
    r.R = sc.R;
    r.iters = a->iters;
    r.spin_limit = spin_limit();
    r.local_ok = local_exchange_allowed();
    r.sweeps = a->sweeps_used;
    r.early = (a->flags & DOT_SK_EXACT_SWEEPS) ? 0 : 1;
    const size_t words = size_t(reinterpret_cast<unsigned long long*>(r.status) - L.pst) + 1;
    const size_t S = (size_t(N) + sc.W - 1) / sc.W;
    bool ok = false;
    dispatch_row(N, vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        // fold rows | mu | red N + W | r, 1/rs, lambda R each | c, cs S each | scratch
        const size_t lds =
            (size_t(pst::kFoldRows<V, C> + 2) * N + sc.W + 3 * size_t(sc.R) + 2 * S + 32) * sizeof(float);
        launch_fill_zero(L.pst, 2 * words, stream);
        ProfScope prof("sk_imp_persistent", stream);
        ok = launch_persistent(pst::implicit_adjoint<V, C>, r, G, res::kThreads, lds, stream);
    });
    if (!ok) return false;
    ProfScope prof("sk_batch_sum", stream);
    hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial, sc.W, -inv_tau,
                       a->grad_tau, static_cast<const int*>(r.status), a->status, 1, keep_status ? 1 : 0);
    return true;
}

// Rows longer than kMaxRowLen: the prologue in chunk tiles with a row-total
// fold, then per sweep a rows pass (chunk partials of P mu), a columns pass
// (lambda and the column partials of P lambda) and the mu combine, then the
// gradient in chunk tiles.
void launch_wide_implicit(const dot_sinkhorn_bwd_args* a, const ImpLayout& L, const sk::ImpArgs& x,
                          float inv_tau, hipStream_t stream) {
    const int B = a->B, M = a->M, N = a->N;
    wide::ImpArgs w{};
    w.s = x;
    w.rpart = L.rpart;
    w.dpart = L.dpart;
    w.B = B;
    w.nchunks = L.nchunks;
    const dim3 tiles = batch_grid(unsigned(L.nstrips) * unsigned(L.nchunks), B);
    const size_t lds = (size_t(2) * wide::kChunk + 8) * sizeof(float);
    const unsigned row_blocks = unsigned((size_t(B) * M + kWavesPerBlock - 1) / kWavesPerBlock);
    wide::dispatch_chunk(bwd_vec4(a), [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        {
            ProfScope prof("sk_imp_prep", stream);
            hipLaunchKernelGGL((wide::imp_prep<V, C>), tiles, dim3(kBlock), lds, stream, w);
        }
        {
            ProfScope prof("sk_imp_prep_combine", stream);
            hipLaunchKernelGGL(wide::imp_row_totals, dim3(row_blocks), dim3(kBlock), 0, stream, w);
            hipLaunchKernelGGL(sk::imp_prep_combine, sk::fold_grid(N, B), dim3(kBlock), 0, stream, x);
        }
        for (int it = 0; it < a->iters; ++it) {
            {
                ProfScope prof("sk_imp_wide_rows", stream);
                hipLaunchKernelGGL((wide::imp_rows<V, C>), tiles, dim3(kBlock), 0, stream, w);
            }
            {
                ProfScope prof("sk_imp_wide_cols", stream);
                hipLaunchKernelGGL((wide::imp_cols<V, C>), tiles, dim3(kBlock), lds, stream, w);
            }
            {
                ProfScope prof("sk_imp_combine", stream);
                hipLaunchKernelGGL(sk::imp_mu_combine, sk::fold_grid(N, B), dim3(kBlock), 0, stream, x);
            }
        }
        {
            ProfScope prof("sk_imp_final", stream);
            hipLaunchKernelGGL((wide::imp_final<V, C>), tiles, dim3(kBlock), 0, stream, w);
        }
        {
            ProfScope prof("sk_batch_sum", stream);
            hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial, int(tiles.x),
                               -inv_tau, a->grad_tau, nullptr, a->status);
        }
    });
}

// The whole reverse pass as one cooperative launch when every batch element
// can have W workgroups (the persistent streaming tier): Gamma and the scores
// are streamed once per step and the column sums of Gamma go through the
// tagged reduce-scatter / all-gather instead of a fold launch per step.
bool launch_stream_unrolled(const dot_sinkhorn_bwd_args* a, const UnrLayout& L, const StreamCfg& sc,
                            float inv_tau, float neg_inv_tau2, bool vec4, hipStream_t stream) {
    const int B = a->B, N = a->N, G = B * sc.W;
    if (!L.pst || size_t(G) > L.pst_groups) return false;
    pst::UnrArgs r{};
    r.X = a->scores;
    r.scores_kind = a->scores_kind;
    r.kscale = float(a->scores_kind) * inv_tau;
    r.gP = a->grad_plan;
    r.gC = a->grad_cost;
    r.gc_step = (a->flags & DOT_SK_GRAD_COST_SCALAR) ? 0 : 1;
    r.P = a->plan;
    r.u_hist = a->u_hist;
    r.v_hist = a->v_hist;
    r.gamma = L.gamma;
    r.part = L.pst;
    r.res = r.part + 2 * size_t(G) * N;
    r.status = reinterpret_cast<int*>(r.res + 2 * size_t(B) * N);
    r.grad = a->grad_scores;
    r.tau_partial = L.tau_partial;
    r.inv_tau = inv_tau;
    r.B = B;
    r.M = a->M;
    r.N = N;
    r.W = sc.W;
    r.R = sc.R;
    r.T = a->iters;
    r.spin_limit = spin_limit();
    r.local_ok = local_exchange_allowed();
    const size_t words = size_t(reinterpret_cast<unsigned long long*>(r.status) - L.pst) + 1;
    bool ok = false;
    dispatch_row(N, vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        // fold rows | colsum | v_t | v_{t-1} N each | red N + W | scratch
        const size_t lds = (size_t(pst::kFoldRows<V, C> + 4) * N + sc.W + 16) * sizeof(float);
        if constexpr (V * C <= 32) {
            launch_fill_zero(L.pst, 2 * words, stream);
            ProfScope prof("sk_unr_persistent", stream);
            ok = launch_persistent(pst::unrolled<V, C>, r, G, res::kThreads, lds, stream);
        } else if constexpr (V == 4 && C == 16) {
            // rows of exactly 4096 floats, streamed in halves through 32-bit
            // buffer offsets (the matrix below 4 GiB); other lengths of 64 floats a
            // lane take the per-step sweeps
            if (N == 4 * C * kWave && size_t(B) * a->M * N * sizeof(float) <= 0xffffffffull) {
                launch_fill_zero(L.pst, 2 * words, stream);
                ProfScope prof("sk_unr_persistent", stream);
                ok = launch_persistent(pst::unrolled_halves<C / 2, true>, r, G, res::kThreads, lds, stream);
            }
        }
    });
    if (!ok) return false;
    ProfScope prof("sk_batch_sum", stream);
    hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial, sc.W, neg_inv_tau2,
                       a->grad_tau, static_cast<const int*>(r.status), a->status);
    return true;
}

// Rows longer than kMaxRowLen: Gamma = G P in chunk tiles, then per recorded
// step the column fold, a rows pass (chunk partials of rowsum(Gamma_Y)) and a
// columns pass (Gamma, or the gradient on the last step).
void launch_wide_unrolled(const dot_sinkhorn_bwd_args* a, const UnrLayout& L, const sk::UnrArgs& x0,
                          float neg_inv_tau2, hipStream_t stream) {
    const int B = a->B, M = a->M, N = a->N, T = a->iters;
    wide::UnrArgs w{};
    w.s = x0;
    w.tpart = L.tpart;
    w.B = B;
    w.nchunks = L.nchunks;
    const dim3 tiles = batch_grid(unsigned(L.nstrips) * unsigned(L.nchunks), B);
    const size_t lds = (size_t(2) * wide::kChunk + 8) * sizeof(float);
    wide::dispatch_chunk(bwd_vec4(a), [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        w.s.final_step = T == 0;
        {
            ProfScope prof("sk_unr_init", stream);
            hipLaunchKernelGGL((wide::unr_init<V, C>), tiles, dim3(kBlock), lds, stream, w);
        }
        for (int t = T - 1; t >= 0; --t) {
            {
                ProfScope prof("sk_unr_fold", stream);
                hipLaunchKernelGGL(sk::column_fold, sk::fold_grid(N, B), dim3(kBlock), 0, stream, L.partial,
                                   L.nstrips, B, N, L.colsum);
            }
            w.s.u_t = a->u_hist + size_t(t) * B * M;
            w.s.v_t = a->v_hist + size_t(t) * B * N;
            w.s.v_tm1 = t > 0 ? a->v_hist + size_t(t - 1) * B * N : nullptr;
            w.s.final_step = t == 0;
            {
                ProfScope prof("sk_unr_wide_rows", stream);
                hipLaunchKernelGGL((wide::unr_rows<V, C>), tiles, dim3(kBlock), 0, stream, w);
            }
            {
                ProfScope prof("sk_unr_step", stream);
                hipLaunchKernelGGL((wide::unr_cols<V, C>), tiles, dim3(kBlock), lds, stream, w);
            }
        }
        {
            ProfScope prof("sk_batch_sum", stream);
            hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial, int(tiles.x),
                               neg_inv_tau2, a->grad_tau, nullptr, a->status);
        }
    });
}

}  // namespace

extern "C" size_t dot_sinkhorn_backward_implicit_workspace_bytes(int B, int M, int N) {
    if (B < 0 || M < 0 || N < 0) return 0;
    return imp_layout(nullptr, B, M, N).bytes;
}

extern "C" int dot_sinkhorn_backward_implicit(const dot_sinkhorn_bwd_args* a, dot_stream_t stream_) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (int rc = check_bwd(a)) return rc;
    const int B = a->B, M = a->M, N = a->N;
    if (size_t(B) * M * N == 0) {
        report_all_sweeps(a, stream);
        return bwd_degenerate(a, stream, "dot_sinkhorn_backward_implicit");
    }
    const ImpLayout L = imp_layout(a->workspace, B, M, N);
    if (!a->workspace || a->workspace_bytes < L.bytes)
        return fail(DOT_ERR_WORKSPACE,
                    "workspace smaller than dot_sinkhorn_backward_implicit_workspace_bytes()");
    const float inv_tau = 1.0f / a->tau;
    sk::ImpArgs x{};
    x.g = grad_source(a);
    x.P = a->plan;
    x.r = L.r;
    x.rs = L.rs;
    x.lam = L.lam;
    x.c = L.c;
    x.cs = L.cs;
    x.mu = L.mu;
    x.partA = L.partA;
    x.partB = L.partB;
    x.nstrips = L.nstrips;
    x.grad = a->grad_scores;
    x.tau_partial = L.tau_partial;
    x.inv_tau = inv_tau;
    x.B = B;
    x.M = M;
    x.N = N;
    x.rows = L.rows;
    const size_t lds = lds_bytes(N);
    const dim3 strips = batch_grid(unsigned(L.nstrips), B);
    const ResidentCfg rc = resident_config<false>(B, M, N, bwd_vec4(a));
    if (rc.ok && launch_resident_adjoint(a, L, rc, inv_tau, stream))
        return check_launch("dot_sinkhorn_backward_implicit");
    (void)hipGetLastError();  // a refused launch falls back to the next tier
    if (!rc.ok) {
        const int slab = resident_slab(B, M, N, bwd_vec4(a));
        if (slab > 0 && slab < B) {
            if (launch_resident_slabs(a, L, slab, inv_tau, stream))
                return check_launch("dot_sinkhorn_backward_implicit");
            if (int e = check_launch("dot_sinkhorn_backward_implicit")) return e;
            (void)hipGetLastError();
        }
    }
    const StreamCfg sc = stream_config(B, M, N);
    if (sc.ok && launch_stream_adjoint(a, L, sc, inv_tau, bwd_vec4(a), stream))
        return check_launch("dot_sinkhorn_backward_implicit");
    (void)hipGetLastError();
    // More elements than CUs: slabs of one element per CU on the persistent tier.
    const int cus = device_cus();
    if (!sc.ok && cus > 0 && B > cus && stream_config(cus, M, N).ok) {
        const bool done = launch_slabs(a, cus, [&](const dot_sinkhorn_bwd_args& s, bool keep) {
            const StreamCfg ss = stream_config(s.B, M, N);
            return ss.ok && launch_stream_adjoint(&s, L, ss, inv_tau, bwd_vec4(&s), stream, keep);
        });
        if (done) return check_launch("dot_sinkhorn_backward_implicit");
        if (int e = check_launch("dot_sinkhorn_backward_implicit")) return e;
        (void)hipGetLastError();
    }
    report_all_sweeps(a, stream);  // the per-sweep launches run every sweep
    if (L.nchunks > 1) {
        launch_wide_implicit(a, L, x, inv_tau, stream);
        return check_launch("dot_sinkhorn_backward_implicit");
    }
    bool launched = dispatch_row(N, bwd_vec4(a), [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        {
            ProfScope prof("sk_imp_prep", stream);
            hipLaunchKernelGGL((sk::imp_prep<V, C>), strips, dim3(kBlock), lds, stream, x);
        }
        {
            ProfScope prof("sk_imp_prep_combine", stream);
            hipLaunchKernelGGL(sk::imp_prep_combine, sk::fold_grid(N, B), dim3(kBlock), 0, stream, x);
        }
        for (int it = 0; it < a->iters; ++it) {
            {
                ProfScope prof("sk_imp_sweep", stream);
                hipLaunchKernelGGL((sk::imp_lambda_sweep<V, C>), strips, dim3(kBlock), lds, stream, x);
            }
            {
                ProfScope prof("sk_imp_combine", stream);
                hipLaunchKernelGGL(sk::imp_mu_combine, sk::fold_grid(N, B), dim3(kBlock), 0, stream, x);
            }
        }
        {
            ProfScope prof("sk_imp_final", stream);
            hipLaunchKernelGGL((sk::imp_final<V, C>), strips, dim3(kBlock), 0, stream, x);
        }
        {
            ProfScope prof("sk_batch_sum", stream);
            hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial,
                               L.nstrips, -inv_tau, a->grad_tau, nullptr, a->status);
        }
    });
    if (!launched) return fail(DOT_ERR_UNSUPPORTED, "row length outside the supported range");
    return check_launch("dot_sinkhorn_backward_implicit");
}

extern "C" size_t dot_sinkhorn_backward_unrolled_workspace_bytes(int B, int M, int N) {
    if (B < 0 || M < 0 || N < 0) return 0;
    return unr_layout(nullptr, B, M, N).bytes;
}

extern "C" int dot_sinkhorn_backward_unrolled(const dot_sinkhorn_bwd_args* a, dot_stream_t stream_) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (int rc = check_bwd(a)) return rc;
    const int B = a->B, M = a->M, N = a->N, T = a->iters;
    if (size_t(B) * M * N == 0) return bwd_degenerate(a, stream, "dot_sinkhorn_backward_unrolled");
    if (T > 0 && (!a->u_hist || !a->v_hist))
        return fail(DOT_ERR_INVALID_ARG, "u_hist and v_hist are required when iters > 0");
    const UnrLayout L = unr_layout(a->workspace, B, M, N);
    if (!a->workspace || a->workspace_bytes < L.bytes)
        return fail(DOT_ERR_WORKSPACE,
                    "workspace smaller than dot_sinkhorn_backward_unrolled_workspace_bytes()");
    const float tau = a->tau;
    const float inv_tau = 1.0f / tau;
    const float neg_inv_tau2 = -1.0f / (tau * tau);  // kernels.cu:1642
    sk::UnrArgs x{};
    x.g = grad_source(a);
    x.kscale = float(a->scores_kind) * inv_tau;
    x.P = a->plan;
    x.gamma = L.gamma;
    x.partial = L.partial;
    x.nstrips = L.nstrips;
    x.colsum = L.colsum;
    x.grad = a->grad_scores;
    x.tau_partial = L.tau_partial;
    x.inv_tau = inv_tau;
    x.B = B;
    x.M = M;
    x.N = N;
    x.rows = L.rows;
    const size_t lds = lds_bytes(N);
    const dim3 strips = batch_grid(unsigned(L.nstrips), B);
    const StreamCfg sc = stream_config(B, M, N);
    if (sc.ok && launch_stream_unrolled(a, L, sc, inv_tau, neg_inv_tau2, bwd_vec4(a), stream))
        return check_launch("dot_sinkhorn_backward_unrolled");
    (void)hipGetLastError();  // a refused cooperative launch falls back to the per-step sweeps
    if (L.nchunks > 1) {
        launch_wide_unrolled(a, L, x, neg_inv_tau2, stream);
        return check_launch("dot_sinkhorn_backward_unrolled");
    }
    bool launched = dispatch_row(N, bwd_vec4(a), [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        x.final_step = T == 0;
        {
            ProfScope prof("sk_unr_init", stream);
            hipLaunchKernelGGL((sk::unr_init<V, C>), strips, dim3(kBlock), lds, stream, x);
        }
        for (int t = T - 1; t >= 0; --t) {
            {
                ProfScope prof("sk_unr_fold", stream);
                hipLaunchKernelGGL(sk::column_fold, sk::fold_grid(N, B), dim3(kBlock), 0, stream,
                                   L.partial, L.nstrips, B, N, L.colsum);
            }
            x.u_t = a->u_hist + size_t(t) * B * M;
            x.v_t = a->v_hist + size_t(t) * B * N;
            x.v_tm1 = t > 0 ? a->v_hist + size_t(t - 1) * B * N : nullptr;
            x.final_step = t == 0;
            {
                ProfScope prof("sk_unr_step", stream);
                hipLaunchKernelGGL((sk::unr_step<V, C>), strips, dim3(kBlock), lds, stream, x);
            }
        }
        {
            ProfScope prof("sk_batch_sum", stream);
            hipLaunchKernelGGL(sk::batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial,
                               L.nstrips, neg_inv_tau2, a->grad_tau, nullptr, a->status);
        }
    });
    if (!launched) return fail(DOT_ERR_UNSUPPORTED, "row length outside the supported range");
    return check_launch("dot_sinkhorn_backward_unrolled");
}

// The allocation-free forward (dot_sinkhorn_forward_noalloc) is in noalloc.hip.
size_t dot_amd::forward_workspace_base_bytes(int B, int M, int N, int max_iter) {
    if (B < 0 || M < 0 || N < 0 || max_iter < 0) return 0;
    return fwd_layout(nullptr, B, M, N, max_iter).bytes;
}
