// Accelerated / scheduled dual Sinkhorn C ABI: argument checks, workspace
// layout and the per-iteration launch sequence.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>
#include <type_traits>
#include <vector>

#include "host.hpp"
#include "methods.cuh"

namespace dot_amd {
namespace {

using mth::kMaxHistory;
using mth::kIterWords;

constexpr int kStopCheckEvery = 16;  // iterations between host reads of the stop flag (tol > 0)

struct MethodLayout {
    unsigned* slots;              // [T, kIterWords] flag words
    float *m1u, *m2u, *m1v, *m2v; // Adam moments
    float *u, *v;                 // final potentials (Anderson: the state)
    size_t zero_bytes;            // from `slots` through `v`
    float *ut[2], *un[2], *vt[2], *vn[2];  // per iteration, by parity
    float *part_t, *part_n, *cost_partial;
    float *hxu, *hxv, *hfu, *hfv, *dots, *gram, *alpha, *denom;
    // rows longer than kMaxRowLen (nchunks > 1): chunk partials and row terms
    float2* rpart;                // [B, nchunks, M]
    float *row_m, *row_w, *row_w2;  // [B, M]
    int rows, nstrips, nchunks;
    size_t bytes;
};

// Rows per sweep workgroup: 32, halved (down to 4) while the grid has fewer
// than 512 workgroups.  A solver sweep carries two column sums and adds its
// flag maxima with atomics, so its per-workgroup cost is higher than the
// vanilla sweep's: measured per momentum iteration, C4 (16 x 1024 x 2048)
// 43 µs at 16 rows, 36 at 32, 39 at 64; C3 (64 x 512 x 512) 24.7 at 32, 27.7
// at 64.  DOT_AMD_ROWS overrides it (tuning only).
int solver_strip_rows(int B, int M) {
    if (const char* s = std::getenv("DOT_AMD_ROWS"))
        if (std::atoi(s) >= 1) return std::atoi(s);
    int r = 32;
    while (r > 4 && int64_t(B) * ((M + r - 1) / r) < 512) r /= 2;
    return r;
}

MethodLayout method_layout(void* ws, int B, int M, int N, int T, int method, int k) {
    Carver c(ws);
    MethodLayout L{};
    // rows longer than a wave's registers run on the strips x chunks tiling
    L.nchunks = N > kMaxRowLen ? wide::num_chunks(N) : 1;
    L.rows = L.nchunks > 1 ? wide::strip_rows(B, M, L.nchunks) : solver_strip_rows(B, M);
    L.nstrips = M > 0 ? (M + L.rows - 1) / L.rows : 0;
    const size_t BM = size_t(B) * M, BN = size_t(B) * N;
    const bool adam = method == DOT_SK_ADAM, anderson = method == DOT_SK_ANDERSON;
    const bool cand = method == DOT_SK_MOMENTUM || adam;
    L.slots = c.take<unsigned>(size_t(std::max(T, 1)) * kIterWords);
    L.m1u = c.take<float>(adam ? BM : 0);
    L.m2u = c.take<float>(adam ? BM : 0);
    L.m1v = c.take<float>(adam ? BN : 0);
    L.m2v = c.take<float>(adam ? BN : 0);
    L.u = c.take<float>(BM);
    L.v = c.take<float>(BN);
    L.zero_bytes = c.used();
    const int parities = anderson ? 1 : 2;
    for (int p = 0; p < 2; ++p) {
        L.ut[p] = p < parities ? c.take<float>(BM) : L.ut[0];
        L.vt[p] = p < parities ? c.take<float>(BN) : L.vt[0];
        L.un[p] = cand ? c.take<float>(BM) : L.ut[p];
        L.vn[p] = cand ? c.take<float>(BN) : L.vt[p];
    }
    L.part_t = c.take<float>(size_t(B) * L.nstrips * N);
    L.part_n = cand ? c.take<float>(size_t(B) * L.nstrips * N) : L.part_t;
    L.cost_partial = c.take<float>(size_t(B) * L.nstrips * L.nchunks);
    const bool wide_rows = L.nchunks > 1;
    L.rpart = c.take<float2>(wide_rows ? size_t(B) * L.nchunks * M : 0);
    L.row_m = c.take<float>(wide_rows ? BM : 0);
    L.row_w = c.take<float>(wide_rows ? BM : 0);
    L.row_w2 = c.take<float>(wide_rows && cand ? BM : 0);
    const size_t kk = anderson ? size_t(k) : 0;
    L.hxu = c.take<float>(kk * BM);
    L.hxv = c.take<float>(kk * BN);
    L.hfu = c.take<float>(kk * BM);
    L.hfv = c.take<float>(kk * BN);
    const size_t nchunk = (size_t(M) + N + mth::kGramChunk - 1) / mth::kGramChunk;
    L.dots = c.take<float>(kk ? size_t(B) * nchunk * kMaxHistory : 0);
    L.gram = c.take<float>(kk ? size_t(B) * kMaxHistory * kMaxHistory : 0);
    L.alpha = c.take<float>(kk ? size_t(B) * kMaxHistory : 0);
    L.denom = c.take<float>(kk ? size_t(B) : 0);
    L.bytes = c.used();
    return L;
}

// tau at iteration `step` of `total` (scheduled_tau_cuda, torch_cuda.cpp:61-84),
// in float as there.
float scheduled_tau(int64_t step, int64_t total, float tau, float reg_start, int schedule) {
    constexpr float kPi = 3.14159265358979323846f;
    if (schedule == DOT_SK_SCHEDULE_NONE || total <= 1) return tau;
    const float start = reg_start > 0.0f ? reg_start : 10.0f * tau;
    const float frac = static_cast<float>(step) / static_cast<float>(total - 1);
    switch (schedule) {
        case DOT_SK_SCHEDULE_LINEAR: return start * (1.0f - frac) + tau * frac;
        case DOT_SK_SCHEDULE_COSINE: return tau + 0.5f * (start - tau) * (1.0f + std::cos(kPi * frac));
        case DOT_SK_SCHEDULE_EXPONENTIAL: return tau * std::pow(start / tau, 1.0f - frac);
        default: return tau;
    }
}

dim3 vector_grid(size_t n) { return dim3(unsigned(std::max<size_t>(1, std::min<size_t>((n + kBlock - 1) / kBlock, 1024)))); }

__global__ void set_counts_m(int32_t* used, int32_t* converged, int u, int c) {
    *used = u;
    *converged = c;
}

__global__ void fill_value_m(float* p, size_t n, float x) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        p[i] = x;
}

__global__ void zero_words(uint32_t* p, size_t n) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        p[i] = 0u;
}

__global__ void batch_sum_m(const float* partial, int n, float* out) {
    // one wave per batch element; strips summed lane-strided then across the wave
    const int b = blockIdx.x;
    float s = 0.0f;
    for (int k = threadIdx.x; k < n; k += kWave) s += partial[size_t(b) * n + k];
    s = wave_sum(s);
    if (threadIdx.x == 0) out[b] = s;
}

// The per-iteration K scales of a schedule reach the device as kernel
// arguments, kTableChunk at a time (no host buffer has to outlive the call).
constexpr int kTableChunk = 256;
struct TableChunk {
    float v[kTableChunk];
};

__global__ void fill_table(float* dst, TableChunk c, int n) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
#pragma unroll
    for (int i = 0; i < kTableChunk; ++i)
        if (i < n) dst[i] = c.v[i];
}

// Workspace of the vanilla method (plain or scheduled): the K-scale table,
// then dot_sinkhorn_forward's workspace.
size_t vanilla_table_bytes(int T) { return (size_t(T) * sizeof(float) + 255) & ~size_t(255); }

// Pairs the Anderson ring holds: the reference keeps the last anderson_k
// (torch_cuda.cpp:395-420), and a run of max_iter iterations pushes at most
// max_iter, so a ring of min(anderson_k, max_iter) never drops one the
// reference would keep.
int ring_pairs(int anderson_k, int max_iter) { return std::max(1, std::min(anderson_k, max_iter)); }

int check_method_args(const dot_sinkhorn_method_args* m) {
    if (m->method < DOT_SK_VANILLA || m->method > DOT_SK_ADAM)
        return fail(DOT_ERR_INVALID_ARG, "method must be 0 (vanilla), 1 (momentum), 2 (anderson) or 3 (adam)");
    if (m->schedule < DOT_SK_SCHEDULE_NONE || m->schedule > DOT_SK_SCHEDULE_COSINE)
        return fail(DOT_ERR_INVALID_ARG, "schedule must be 0 (none), 1 (linear), 2 (exponential) or 3 (cosine)");
    if (m->anderson_k < 1) return fail(DOT_ERR_INVALID_ARG, "anderson_k must be >= 1");
    if (m->method == DOT_SK_ANDERSON && ring_pairs(m->anderson_k, m->base.max_iter) > kMaxHistory)
        return fail(DOT_ERR_UNSUPPORTED, "Anderson histories longer than " + std::to_string(kMaxHistory) +
                                              " pairs (anderson_k and max_iter both above it) are not "
                                              "supported by this build");
    return DOT_OK;
}

}  // namespace
}  // namespace dot_amd

using namespace dot_amd;

extern "C" size_t dot_sinkhorn_forward_method_workspace_bytes(int B, int M, int N, int max_iter, int method,
                                                              int anderson_k) {
    if (B < 0 || M < 0 || N < 0 || max_iter < 0 || anderson_k < 0) return 0;
    if (method == DOT_SK_VANILLA)
        return vanilla_table_bytes(max_iter) + dot_sinkhorn_forward_workspace_bytes(B, M, N, max_iter, 0);
    return method_layout(nullptr, B, M, N, max_iter, method, std::min(ring_pairs(anderson_k, max_iter), kMaxHistory))
        .bytes;
}

extern "C" int dot_sinkhorn_forward_method(const dot_sinkhorn_method_args* m, dot_stream_t stream_) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (!m) return fail(DOT_ERR_INVALID_ARG, "args is NULL");
    const dot_sinkhorn_fwd_args* a = &m->base;
    const int B = a->B, M = a->M, N = a->N, T = a->max_iter;
    if (B < 0 || M < 0 || N < 0) return fail(DOT_ERR_INVALID_ARG, "B, M and N must be >= 0");
    if (!(std::isfinite(a->tau) && a->tau > 0.0f)) return fail(DOT_ERR_INVALID_ARG, "tau must be > 0");
    if (T < 0) return fail(DOT_ERR_INVALID_ARG, "max_iter must be >= 0");
    if (a->scores_kind != DOT_SCORES_LOG_ALPHA && a->scores_kind != DOT_SCORES_COST)
        return fail(DOT_ERR_INVALID_ARG, "scores_kind must be DOT_SCORES_LOG_ALPHA or DOT_SCORES_COST");
    if (!a->iters_used || !a->converged)
        return fail(DOT_ERR_INVALID_ARG, "iters_used and converged must be device pointers");
    if (a->flags & ~DOT_SK_RETURN_LOG)
        return fail(DOT_ERR_INVALID_ARG, "only DOT_SK_RETURN_LOG is accepted by dot_sinkhorn_forward_method");
    const bool ret_log = (a->flags & DOT_SK_RETURN_LOG) != 0;
    if (ret_log && a->cost) return fail(DOT_ERR_INVALID_ARG, "cost is undefined with DOT_SK_RETURN_LOG");
    if (int rc = check_method_args(m)) return rc;
    const int method = m->method;
    const bool sched = m->schedule != DOT_SK_SCHEDULE_NONE;
    const bool track = a->tol > 0.0f;

    const size_t elems = size_t(B) * M * N;
    if (elems == 0) {
        // as the vanilla entry point: an empty delta is 0, so tol > 0 stops at t = 1
        const bool stop = track && T > 0;
        hipLaunchKernelGGL(set_counts_m, dim3(1), dim3(1), 0, stream, a->iters_used, a->converged,
                           stop ? 1 : T, stop ? 1 : 0);
        if (a->cost && B > 0)
            hipLaunchKernelGGL(fill_value_m, dim3(1), dim3(kBlock), 0, stream, a->cost, size_t(B), 0.0f);
        if (a->u_out && size_t(B) * M)
            hipLaunchKernelGGL(fill_value_m, dim3(1), dim3(kBlock), 0, stream, a->u_out, size_t(B) * M, 0.0f);
        if (a->v_out && size_t(B) * N)
            hipLaunchKernelGGL(fill_value_m, dim3(1), dim3(kBlock), 0, stream, a->v_out, size_t(B) * N, 0.0f);
        return check_launch("dot_sinkhorn_forward_method");
    }
    if (!a->scores) return fail(DOT_ERR_INVALID_ARG, "scores is NULL");

    const float tau = a->tau;
    const float sign = static_cast<float>(a->scores_kind);
    auto kscale_at = [&](float t) { return sign * (1.0f / t); };  // kernels.cu:1350 (K = log_alpha * (1/tau))

    if (method == DOT_SK_VANILLA) {
        // The plain iteration, scheduled or not, runs on dot_sinkhorn_forward's
        // tiers with each iteration's K scale (sinkhorn_dual_vanilla_cuda,
        // torch_cuda.cpp:147-264: K rebuilt at every iteration's tau).
        const size_t tb = vanilla_table_bytes(sched ? T : 0);
        if (!a->workspace || a->workspace_bytes < tb)
            return fail(DOT_ERR_WORKSPACE, "workspace smaller than dot_sinkhorn_forward_method_workspace_bytes()");
        dot_sinkhorn_fwd_args f = *a;
        f.workspace = static_cast<char*>(a->workspace) + tb;
        f.workspace_bytes = a->workspace_bytes - tb;
        if (!sched) return sinkhorn_forward_scheduled(&f, nullptr, nullptr, stream);
        std::vector<float> ks(static_cast<size_t>(T));
        for (int t = 0; t < T; ++t) ks[t] = kscale_at(scheduled_tau(t, T, tau, m->reg_start, m->schedule));
        float* table = static_cast<float*>(a->workspace);
        for (int t0 = 0; t0 < T; t0 += kTableChunk) {
            TableChunk c{};
            const int n = std::min(kTableChunk, T - t0);
            std::copy(ks.begin() + t0, ks.begin() + t0 + n, c.v);
            hipLaunchKernelGGL(fill_table, dim3(1), dim3(kWave), 0, stream, table + t0, c, n);
        }
        if (int rc = check_launch("dot_sinkhorn_forward_method (K-scale table)")) return rc;
        return sinkhorn_forward_scheduled(&f, ks.data(), table, stream);
    }

    const int k = ring_pairs(m->anderson_k, T);  // <= kMaxHistory (checked)
    const MethodLayout L = method_layout(a->workspace, B, M, N, T, method, k);
    if (!a->workspace || a->workspace_bytes < L.bytes)
        return fail(DOT_ERR_WORKSPACE, "workspace smaller than dot_sinkhorn_forward_method_workspace_bytes()");

    const float log_a_default = -std::log(static_cast<float>(M));  // torch_cuda.cpp:42
    const float log_b_default = -std::log(static_cast<float>(N));
    const bool vec4 = (N % 4 == 0) && aligned16(a->scores) && (!a->plan || aligned16(a->plan));
    const size_t BM = size_t(B) * M, BN = size_t(B) * N;

    // capture-safe fill kernel instead of a memset node
    {
        const size_t words = L.zero_bytes / sizeof(uint32_t);
        hipLaunchKernelGGL(zero_words, vector_grid(words), dim3(kBlock), 0, stream,
                           reinterpret_cast<uint32_t*>(L.slots), words);
        hipLaunchKernelGGL(mth::reset_counts, dim3(1), dim3(1), 0, stream, a->iters_used, a->converged);
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) cap = hipStreamCaptureStatusNone;
    (void)hipGetLastError();
    const bool may_wait = track && cap == hipStreamCaptureStatusNone;
    const bool anderson = method == DOT_SK_ANDERSON;

    int rc = DOT_OK;
    // V, C: the row layout (a whole row, or one kChunk tile of it when WIDE)
    auto body = [&](auto vc, auto cc, auto wide_c) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        constexpr bool WIDE = decltype(wide_c)::value;
        const dim3 strips = batch_grid(unsigned(L.nstrips * L.nchunks), B);  // strips x chunks tiles
        const dim3 cols = batch_grid(unsigned((N + mth::kFoldCols - 1) / mth::kFoldCols), B);
        const size_t sweep_lds = (size_t(2) * (WIDE ? wide::kChunk : N) + 16) * sizeof(float);  // columns + flags
        int ring_head = 0, ring_size = 0;  // Anderson ring: logical position -> physical slot

        auto iteration = [&](auto mode_c, int t, float ks) {
            constexpr int MODE = decltype(mode_c)::value;
            const unsigned* prev = t > 0 ? L.slots + size_t(t - 1) * kIterWords : nullptr;
            unsigned* cur = L.slots + size_t(t) * kIterWords;
            const int p = t & 1, q = p ^ 1;
            float c1 = 1.0f, c2 = 1.0f;
            if (method == DOT_SK_ADAM && m->bias_correction) {  // torch_cuda.cpp:478-481
                c1 = 1.0f - std::pow(m->beta1, static_cast<float>(t + 1));
                c2 = 1.0f - std::pow(m->beta2, static_cast<float>(t + 1));
            }
            mth::SweepArgs sa{};
            sa.X = a->scores;
            sa.kscale = ks;
            sa.B = B;
            sa.M = M;
            sa.N = N;
            sa.rows = L.rows;
            sa.nstrips = L.nstrips;
            sa.log_a = a->log_a;
            sa.log_a_default = log_a_default;
            if (anderson) {
                sa.u_prev[0] = sa.u_prev[1] = L.u;
                sa.v_prev[0] = sa.v_prev[1] = L.v;
            } else if (t > 0) {
                sa.u_prev[0] = L.ut[q];
                sa.u_prev[1] = L.un[q];
                sa.v_prev[0] = L.vt[q];
                sa.v_prev[1] = L.vn[q];
            }
            sa.prev = prev;
            sa.slots = cur;
            sa.method = method;
            sa.tol = a->tol;
            sa.track = track && method == DOT_SK_VANILLA ? 1 : 0;
            sa.ut = L.ut[p];
            sa.un = L.un[p];
            sa.m1 = L.m1u;
            sa.m2 = L.m2u;
            sa.omega = m->omega;
            sa.lr = m->lr;
            sa.beta1 = m->beta1;
            sa.beta2 = m->beta2;
            sa.c1 = c1;
            sa.c2 = c2;
            sa.eps = m->eps_adam;
            sa.part_t = L.part_t;
            sa.part_n = L.part_n;
            sa.t = t;
            sa.used = a->iters_used;
            sa.converged = a->converged;
            if constexpr (WIDE) {
                mth::WideArgs wa{};
                wa.s = sa;
                wa.nchunks = L.nchunks;
                wa.rpart = L.rpart;
                wa.row_m = L.row_m;
                wa.row_w = L.row_w;
                wa.row_w2 = L.row_w2;
                const int fin_rows = kWavesPerBlock * mth::kFinishRowsPerWave;
                ProfScope prof("mth_sweep", stream);
                hipLaunchKernelGGL((mth::wide_rows<V, C, MODE>), strips, dim3(kBlock), 0, stream, wa);
                hipLaunchKernelGGL((mth::wide_finish<MODE>), batch_grid(unsigned((M + fin_rows - 1) / fin_rows), B),
                                   dim3(kBlock), 0, stream, wa);
                hipLaunchKernelGGL((mth::wide_cols<V, C, MODE>), strips, dim3(kBlock), sweep_lds, stream, wa);
            } else {
                ProfScope prof("mth_sweep", stream);
                hipLaunchKernelGGL((mth::sweep<V, C, MODE>), strips, dim3(kBlock), sweep_lds, stream, sa);
            }
            mth::VfinishArgs fa{};
            fa.X = a->scores;
            fa.kscale = ks;
            fa.B = B;
            fa.M = M;
            fa.N = N;
            fa.nstrips = L.nstrips;
            fa.log_b = a->log_b;
            fa.log_b_default = log_b_default;
            fa.v_prev[0] = sa.v_prev[0];
            fa.v_prev[1] = sa.v_prev[1];
            fa.ut = L.ut[p];
            fa.un = L.un[p];
            fa.prev = prev;
            fa.slots = cur;
            fa.method = method;
            fa.tol = a->tol;
            fa.part_t = L.part_t;
            fa.part_n = L.part_n;
            fa.vt = L.vt[p];
            fa.vn = L.vn[p];
            fa.m1 = L.m1v;
            fa.m2 = L.m2v;
            fa.omega = m->omega;
            fa.lr = m->lr;
            fa.beta1 = m->beta1;
            fa.beta2 = m->beta2;
            fa.c1 = c1;
            fa.c2 = c2;
            fa.eps = m->eps_adam;
            {
                ProfScope prof("mth_vfinish", stream);
                hipLaunchKernelGGL((mth::vfinish<MODE>), cols, dim3(kBlock), 0, stream, fa);
            }
            if (!anderson) return;
            // x_new = (u*, v*); mix the state (torch_cuda.cpp:395-446)
            int slot;
            if (ring_size < k) {
                slot = (ring_head + ring_size) % k;
                ++ring_size;
            } else {
                slot = ring_head;
                ring_head = (ring_head + 1) % k;
            }
            mth::AaArgs aa{};
            aa.B = B;
            aa.M = M;
            aa.N = N;
            aa.xu = L.u;
            aa.xv = L.v;
            aa.nu = L.ut[0];
            aa.nv = L.vt[0];
            aa.hxu = L.hxu;
            aa.hxv = L.hxv;
            aa.hfu = L.hfu;
            aa.hfv = L.hfv;
            aa.slot = slot;
            aa.h = ring_size;
            for (int c = 0; c < ring_size; ++c) aa.order[c] = (ring_head + c) % k;
            aa.mixing_beta = m->mixing_beta;
            aa.dots = L.dots;
            aa.gram = L.gram;
            aa.nchunk = (M + N + mth::kGramChunk - 1) / mth::kGramChunk;
            aa.alpha = L.alpha;
            aa.denom = L.denom;
            aa.prev = prev;
            aa.slots = cur;
            aa.tol = a->tol;
            ProfScope prof("mth_anderson", stream);
            hipLaunchKernelGGL(mth::aa_push, batch_grid(unsigned(aa.nchunk), B), dim3(kBlock), 0, stream, aa);
            hipLaunchKernelGGL(mth::aa_solve, dim3(B), dim3(kBlock), 0, stream, aa);
            hipLaunchKernelGGL(mth::aa_update, vector_grid(BM + BN), dim3(kBlock), 0, stream, aa);
        };

        float ks = kscale_at(scheduled_tau(0, T, tau, m->reg_start, m->schedule));
        for (int t = 0; t < T; ++t) {
            if (sched) ks = kscale_at(scheduled_tau(t, T, tau, m->reg_start, m->schedule));
            switch (method) {
                case DOT_SK_MOMENTUM: iteration(std::integral_constant<int, mth::kMomentum>{}, t, ks); break;
                case DOT_SK_ADAM: iteration(std::integral_constant<int, mth::kAdam>{}, t, ks); break;
                default: iteration(std::integral_constant<int, mth::kPlain>{}, t, ks); break;
            }
            if (may_wait && (t + 1) % kStopCheckEvery == 0 && t + 1 < T) {
                // stop launching once the device's test has fired (an iteration
                // that did not run reads as met, so this one's words suffice)
                unsigned words[kIterWords];
                if (hipMemcpyAsync(words, L.slots + size_t(t) * kIterWords, sizeof(words), hipMemcpyDeviceToHost,
                                   stream) != hipSuccess ||
                    hipStreamSynchronize(stream) != hipSuccess) {
                    rc = check_launch("dot_sinkhorn_forward_method (stop-flag read)");
                    if (rc == DOT_OK) rc = fail(DOT_ERR_HIP, "dot_sinkhorn_forward_method: stop-flag read failed");
                    return;
                }
                if (mth::decide_host(words, method).delta < a->tol) break;
            }
        }
        if (T > 0)
            hipLaunchKernelGGL(mth::finalize, dim3(1), dim3(kWave), 0, stream, L.slots + size_t(T - 1) * kIterWords,
                               method, a->tol, a->converged);
        if (!anderson) {
            mth::ResolveArgs ra{};
            ra.B = B;
            ra.M = M;
            ra.N = N;
            ra.method = method;
            ra.used = a->iters_used;
            ra.slots = L.slots;
            for (int p = 0; p < 2; ++p) {
                ra.ut[p] = L.ut[p];
                ra.un[p] = L.un[p];
                ra.vt[p] = L.vt[p];
                ra.vn[p] = L.vn[p];
            }
            ra.u = L.u;
            ra.v = L.v;
            hipLaunchKernelGGL(mth::resolve, vector_grid(BM + BN), dim3(kBlock), 0, stream, ra);
        }

        // plan and cost at the target tau (torch_cuda.cpp:538-552, :242-261)
        if (a->plan || a->cost) {
            mth::PlanArgs pa{};
            pa.X = a->scores;
            pa.kscale = kscale_at(tau);
            pa.csign = -sign;  // C = -log_alpha
            pa.B = B;
            pa.M = M;
            pa.N = N;
            pa.rows = L.rows;
            pa.nchunks = L.nchunks;
            pa.return_log = ret_log ? 1 : 0;
            pa.safe = method == DOT_SK_VANILLA ? 1 : 0;
            pa.u = L.u;
            pa.v = L.v;
            pa.plan = a->plan;
            pa.cost_partial = a->cost ? L.cost_partial : nullptr;
            ProfScope prof("mth_plan", stream);
            hipLaunchKernelGGL((mth::plan<V, C>), strips, dim3(kBlock), 0, stream, pa);
            if (a->cost)
                hipLaunchKernelGGL(batch_sum_m, dim3(B), dim3(kWave), 0, stream, L.cost_partial,
                                   L.nstrips * L.nchunks, a->cost);
        }
    };
    bool launched = true;
    if (L.nchunks > 1)
        wide::dispatch_chunk(vec4, [&](auto vc, auto cc) { body(vc, cc, std::true_type{}); });
    else
        launched = dispatch_row(N, vec4, [&](auto vc, auto cc) { body(vc, cc, std::false_type{}); });
    if (rc != DOT_OK) return rc;
    if (!launched) return fail(DOT_ERR_UNSUPPORTED, "row length outside the supported range");
    if (a->u_out && hipMemcpyAsync(a->u_out, L.u, BM * sizeof(float), hipMemcpyDeviceToDevice, stream) != hipSuccess)
        return check_launch("dot_sinkhorn_forward_method (u_out)");
    if (a->v_out && hipMemcpyAsync(a->v_out, L.v, BN * sizeof(float), hipMemcpyDeviceToDevice, stream) != hipSuccess)
        return check_launch("dot_sinkhorn_forward_method (v_out)");
    return check_launch("dot_sinkhorn_forward_method");
}
