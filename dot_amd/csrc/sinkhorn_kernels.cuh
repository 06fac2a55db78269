// Sinkhorn device kernels (forward, implicit adjoint, unrolled backward).
//
// Every per-iteration step is one "sweep" over the [B, M, N] matrix in row
// strips: a workgroup of 4 waves owns `rows` consecutive rows of one batch
// element, a wave holds a whole row in registers (row.cuh), reduces it across
// its 64 lanes, and keeps per-column running sums for the rows it visits.
// The workgroup folds its 4 waves' column sums in a fixed order and writes one
// partial row per strip; a small "combine" kernel then folds the strips of a
// batch element into the column update.  Each element is read from HBM once
// per iteration; nothing is reduced with float atomics, so results are
// bitwise reproducible from run to run.
#pragma once

#include <cfloat>
#include <cstdint>

#include "row.cuh"

namespace dot_amd {
namespace sk {

// Column sums below this floor make the shared-exponential column update
// inaccurate; those columns are recomputed with an exact max-shifted LSE.
constexpr float kColSumFloor = 1.0e-20f;
constexpr float kSumFloor = 1.0e-12f;  // log(max(sum, 1e-12)), kernels.cu:538

// Folds of per-strip column partials ([B, nstrips, N]) run kFoldCols columns
// per workgroup with kFoldLanes lanes per column: lane l adds strips l,
// l + kFoldLanes, ... in order, then a fixed halving tree adds the lanes, so
// every column is summed in the same order on every run (one thread per column
// looping over the strips left most of the chip idle).
constexpr int kFoldCols = 16;
constexpr int kFoldLanes = kBlock / kFoldCols;  // 16

inline dim3 fold_grid(int N, int B) { return batch_grid(unsigned((N + kFoldCols - 1) / kFoldCols), B); }

// Column j's sums of NS partial planes; valid in the threads with fold_lane() == 0.
// Every thread of the workgroup must call it (barriers).
__device__ __forceinline__ int fold_lane() { return int(threadIdx.x) / kFoldCols; }
__device__ __forceinline__ int fold_col() { return int(blockIdx.x) * kFoldCols + int(threadIdx.x) % kFoldCols; }

template <int NS>
__device__ __forceinline__ void fold_strips(const float* const (&planes)[NS], int nstrips, int N, int b,
                                            float (&out)[NS]) {
    __shared__ float sm[NS][kFoldLanes][kFoldCols];
    const int jj = int(threadIdx.x) % kFoldCols, sl = fold_lane(), j = fold_col();
#pragma unroll
    for (int q = 0; q < NS; ++q) out[q] = 0.0f;
    if (j < N) {
        const size_t base = size_t(b) * nstrips * N + j;
        for (int k = sl; k < nstrips; k += kFoldLanes)
#pragma unroll
            for (int q = 0; q < NS; ++q) out[q] += planes[q][base + size_t(k) * N];
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) sm[q][sl][jj] = out[q];
#pragma unroll
    for (int half = kFoldLanes / 2; half >= 1; half /= 2) {
        __syncthreads();
        if (sl < half) {
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                out[q] += sm[q][sl + half][jj];
                sm[q][sl][jj] = out[q];
            }
        }
    }
}

// True when the stopping test fired at or before iteration t-1, so iteration
// t must not run.  delta[t] holds the batch-global max|u_t - u_{t-1}| as float
// bits (atomicMax of non-negative floats); iterations that never ran leave 0,
// which chains the stop forward.
__device__ __forceinline__ bool stopped_before(const unsigned* delta_bits, int t, float tol) {
    return tol > 0.0f && t > 1 && __uint_as_float(delta_bits[t - 1]) < tol;
}

// -------------------------------------------------------------------------
// Forward
// -------------------------------------------------------------------------
struct FwdSweepArgs {
    const float* X;        // scores [B,M,N]
    float kscale;          // K = X * kscale (sign/tau)
    const float* log_a;    // [B,M] or null
    float log_a_default;
    const float* v_old;    // [B,N]
    const float* u_old;    // [B,M]
    float* u_new;          // [B,M]
    float* u_hist;         // [B,M] slice of the history for this iteration, or null
    float* partial;        // [B,nstrips,N]
    unsigned* delta_bits;  // [max_iter+1]
    int B, M, N, rows, nstrips, t;
    float tol;
};

// Row update of iteration t fused with the column partial sums it feeds.
//   m_i = max_j(K_ij + v_j), s_i = sum_j exp(K_ij + v_j - m_i),
//   u_i = log a_i - (m_i + log max(s_i, 1e-12))          (kernels.cu:503-545)
// and, sharing the exponentials e_ij = exp(K_ij + v_j - m_i):
//   colsum_j += e_ij * exp(log a_i - log s_i) = exp(K_ij + u_i + v_j),
// so the column update needs no second pass over K:
//   v_j' = log b_j - LSE_i(K_ij + u_i) = log b_j + v_j - log colsum_j.
// The row is reduced in base 2 (y = K log2 e + v log2 e, m = max y,
// s = sum 2^(y - m), u = log a - ln2 (m + log2 s)), the same arithmetic as
// the register-resident and persistent forwards, so that every tier rounds
// u alike and the stop test fires at the same iteration on every tier.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void fwd_sweep(FwdSweepArgs a) {
    if (stopped_before(a.delta_bits, a.t, a.tol)) return;
    using R = Row<VEC, CH>;
    extern __shared__ float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int s = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;

    float v2[R::PL];
    R::load(a.v_old + size_t(b) * a.N, lane, a.N, v2, 0.0f);
    const float kscale2 = a.kscale * kLog2E;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        v2[e] *= kLog2E;
        acc[e] = 0.0f;
    }
    float dmax = 0.0f;

    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (bM + i) * a.N, lane, a.N, x, 0.0f);
        float mloc = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] = R::valid(lane, e, a.N) ? fmaf(x[e], kscale2, v2[e]) : -INFINITY;
            mloc = fmaxf(mloc, x[e]);
        }
        const float m = wave_max(mloc);
        float sloc = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] = __builtin_amdgcn_exp2f(x[e] - m);
            sloc += x[e];
        }
        const float ssum = wave_sum(sloc);
        const float lga = a.log_a ? a.log_a[bM + i] : a.log_a_default;
        const float lg2 = __builtin_amdgcn_logf(fmaxf(ssum, kSumFloor));  // log2
        const float u = lga - kLn2 * (m + lg2);
        const float w = __builtin_amdgcn_exp2f(fmaf(lga, kLog2E, -lg2));  // a / s
#pragma unroll
        for (int e = 0; e < R::PL; ++e) acc[e] = fmaf(x[e], w, acc[e]);
        if (lane == 0) {
            a.u_new[bM + i] = u;
            if (a.u_hist) a.u_hist[bM + i] = u;
            if (a.tol > 0.0f) dmax = fmaxf(dmax, fabsf(u - a.u_old[bM + i]));
        }
    }

    block_column_combine<VEC, CH>(acc, lds, a.N);
    if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + s) * a.N, lane, a.N, acc);
    if (a.tol > 0.0f) {
        const float bm = block_reduce<kWavesPerBlock>(dmax, lds + 2 * a.N, OpMax{});
        if (threadIdx.x == 0) atomicMax(a.delta_bits + a.t, __float_as_uint(bm));
    }
}

struct FwdCombineArgs {
    const float* partial;  // [B,nstrips,N]
    int nstrips;
    const float* X;        // for the exact fallback
    float kscale;
    const float* u_new;    // [B,M]
    const float* log_b;    // [B,N] or null
    float log_b_default;
    const float* v_old;    // [B,N]
    float* v_new;          // [B,N]
    float* v_hist;         // [B,N] slice or null
    const unsigned* delta_bits;
    float tol;
    int t, B, M, N;
};

// Column update v_j = log b_j + v_j - log colsum_j (kernels.cu:629-671 in
// shared-exponential form); columns whose sum is below kColSumFloor (or not
// finite) take the reference's exact max-shifted LSE over the column.
static __global__ __launch_bounds__(kBlock) void fwd_combine(FwdCombineArgs a) {
    if (stopped_before(a.delta_bits, a.t, a.tol)) return;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const float* planes[1] = {a.partial};
    float sum[1];
    fold_strips<1>(planes, a.nstrips, a.N, b, sum);
    const int j = fold_col();
    if (fold_lane() != 0 || j >= a.N) return;
    const float cs = sum[0];
    const size_t bj = size_t(b) * a.N + j;
    const float lgb = a.log_b ? a.log_b[bj] : a.log_b_default;
    float vn;
    if (cs >= kColSumFloor && cs <= FLT_MAX) {
        vn = lgb + a.v_old[bj] - logf(cs);
    } else {
        const float* col = a.X + size_t(b) * a.M * a.N + j;
        const float* u = a.u_new + size_t(b) * a.M;
        float mx = -FLT_MAX;
        for (int i = 0; i < a.M; ++i) mx = fmaxf(mx, col[size_t(i) * a.N] * a.kscale + u[i]);
        float sm = 0.0f;
        for (int i = 0; i < a.M; ++i) sm += safe_exp(col[size_t(i) * a.N] * a.kscale + u[i] - mx);
        vn = lgb - (mx + logf(fmaxf(sm, kSumFloor)));
    }
    a.v_new[bj] = vn;
    if (a.v_hist) a.v_hist[bj] = vn;
}

// Iterations executed and the converged flag, from the per-iteration deltas
// (the host loop's break at torch_cuda.cpp:225-237, evaluated after the fact).
static __global__ void fwd_finalize(const unsigned* delta_bits, int max_iter, float tol,
                             int32_t* iters_used, int32_t* converged) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    int used = max_iter;
    int conv = 0;
    if (tol > 0.0f) {
        for (int t = 1; t <= max_iter; ++t) {
            if (__uint_as_float(delta_bits[t]) < tol) {
                used = t;
                conv = 1;
                break;
            }
        }
    }
    *iters_used = used;
    *converged = conv;
}

struct MaterializeArgs {
    const float* X;
    float kscale;
    int scores_kind;        // +1 log_alpha, -1 cost
    const float* ubuf;      // [2,B,M] double buffer; parity = iters_used & 1
    const float* vbuf;      // [2,B,N]
    const int32_t* iters_used;
    float* plan;            // [B,M,N] or null
    int return_log;
    float* cost_partial;    // [B, gridDim.x] or null
    float* u_out;           // [B,M] or null
    float* v_out;           // [B,N] or null
    int B, M, N, rows;
};

// P = safe_exp(K + u_i + v_j) (kernels.cu:755-775) fused with per-block sums
// of P * C for the transport cost (dot/sinkhorn.py:1703).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void materialize(MaterializeArgs a) {
    using R = Row<VEC, CH>;
    __shared__ float scratch[kWavesPerBlock];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int par = (*a.iters_used) & 1;
    const float* u = a.ubuf + (size_t(par) * a.B + b) * a.M;
    const float* vsrc = a.vbuf + (size_t(par) * a.B + b) * a.N;
    float v[R::PL];
    R::load(vsrc, lane, a.N, v, 0.0f);
    if (a.v_out && blockIdx.x == 0 && wave == 0) R::store(a.v_out + size_t(b) * a.N, lane, a.N, v);
    const int r0 = blockIdx.x * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const float csign = a.scores_kind < 0 ? 1.0f : -1.0f;  // C = -log_alpha
    float cacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (bM + i) * a.N, lane, a.N, x, 0.0f);
        const float ui = u[i];
        float p[R::PL];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float lp = (x[e] * a.kscale + ui) + v[e];
            p[e] = a.return_log ? lp : safe_exp(lp);
            if (a.cost_partial && R::valid(lane, e, a.N)) cacc = fmaf(p[e], csign * x[e], cacc);
        }
        if (a.plan) R::store(a.plan + (bM + i) * a.N, lane, a.N, p);
        if (a.u_out && lane == 0) a.u_out[bM + i] = ui;
    }
    if (a.cost_partial) {
        const float t = block_reduce<kWavesPerBlock>(wave_sum(cacc), scratch, OpSum{});
        if (threadIdx.x == 0) a.cost_partial[size_t(b) * gridDim.x + blockIdx.x] = t;
    }
}

// out[b] = scale * sum_k partial[b, k] in a fixed order; one wave per batch element.
// When status_out is given, block 0 also writes the preceding cooperative
// kernel's status word there (0 when status_in is null): it runs after that
// kernel on the stream, so the word is final.
// status_out (block 0): 1 when *status_in has reached `mark` (the call's
// failure mark, 1 for a status word cleared for the call), else 0.
// Per-element sums of nblk partials; block 0 also turns the exchange status
// into the caller's status word (1 when a wait gave up), or with `keep` raises
// it only, so that a failure of an earlier launch of the call stays visible.
static __global__ void batch_sum(const float* partial, int nblk, float scale, float* out,
                                 const int* status_in = nullptr, int32_t* status_out = nullptr, int mark = 1,
                                 int keep = 0) {
    const int b = blockIdx.x;
    float s = 0.0f;
    for (int k = threadIdx.x; k < nblk; k += kWave) s += partial[size_t(b) * nblk + k];
    s = wave_sum(s);
    if (threadIdx.x == 0) out[b] = s * scale;
    if (status_out && b == 0 && threadIdx.x == 0) {
        const int failed = status_in ? (*status_in >= mark) : 0;
        if (!keep) *status_out = failed;
        else if (failed) *status_out = 1;
    }
}

static __global__ void fill_zero(uint32_t* p, size_t n) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += size_t(gridDim.x) * blockDim.x)
        p[i] = 0u;
}

// fill_zero for a 16-byte aligned p: 16-byte stores, then the last n % 4 words.
static __global__ void fill_zero16(uint32_t* p, size_t n) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    const size_t t = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    uint4* q = reinterpret_cast<uint4*>(p);
    for (size_t i = t; i < n / 4; i += stride) q[i] = make_uint4(0u, 0u, 0u, 0u);
    if (t < n % 4) p[n - n % 4 + t] = 0u;
}

// -------------------------------------------------------------------------
// Upstream gradient of the plan: G = grad_plan + grad_cost[b] * C.
// -------------------------------------------------------------------------
struct GradSource {
    const float* X;
    int scores_kind;
    const float* gP;   // [B,M,N] or null
    const float* gC;   // [B] or null
    int gc_step;       // 1, or 0: gC holds one value for every batch element
};

template <int VEC, int CH>
__device__ __forceinline__ void load_upstream(const GradSource& g, int b, size_t row_off, int lane,
                                              int N, float (&x)[VEC * CH], float (&G)[VEC * CH]) {
    using R = Row<VEC, CH>;
    R::load(g.X + row_off, lane, N, x, 0.0f);
    if (g.gP) {
        R::load(g.gP + row_off, lane, N, G, 0.0f);
    } else {
#pragma unroll
        for (int e = 0; e < R::PL; ++e) G[e] = 0.0f;
    }
    if (g.gC) {
        const float gc = g.gC[b * g.gc_step];
        const float csign = g.scores_kind < 0 ? 1.0f : -1.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) G[e] += gc * (csign * x[e]);
    }
}

// -------------------------------------------------------------------------
// Implicit adjoint
// -------------------------------------------------------------------------

// Early end of the one-launch adjoints (register-resident and persistent
// tiers).  A sweep's lambda_i is a P-weighted average of the previous sweep's
// mu, and its mu_k a P-weighted average of its lambda (plus constants), so
// with d_t = max_k |mu_t - mu_{t-1}| every change of lambda after sweep t is
// at most d_t and, in exact arithmetic, d_{t+1} <= d_t: all later changes of
// lambda_i + mu_k together are at most sum_{j>t} (d_{j-1} + d_j)
// = d_t (1 + rho) / (1 - rho) when the changes shrink by at least rho per
// sweep.  With s_t = max_k (|c_k| + |sum_i P_ik lambda_i|) / cs_k, the size of
// the operands of sweep t's mu update (its fp32 rounding is a few units in
// the last place of s_t), the adjoint ends after sweep t when
//  (a) d_t = 0: mu is a fixed point and every later sweep would repeat this
//      one bit for bit, so the result is exactly the full count's;
//  (b) the last three ratios d_j / d_{j-1} are at most kAdjRhoMax and, with
//      rho their maximum, d_t (1 + rho) / (1 - rho) <= kAdjEps s_t: what the
//      remaining sweeps could still change is below the rounding of the
//      operands; or
//  (c) d_t >= d_{t-1} and d_t <= kAdjFloor s_t: the change did not shrink,
//      which exact arithmetic excludes for a nonzero change (the iteration
//      operator's eigenvalues below 1 are non-negative, and the modes of
//      eigenvalue 1 are constant offsets that never change), so rounding now
//      dominates it: the fp32 sweeps have reached their floor (a rounding
//      cycle) and later sweeps only move within it.
// Slowly contracting problems (ratios above kAdjRhoMax that never reach the
// rounding floor) run every sweep.  d_t and s_t are the same bits in every
// workgroup of a batch element (they all hold the same column sums and mu),
// so the element's workgroups stop together.
constexpr float kAdjRhoMax = 0.5f;
constexpr float kAdjEps = 2.38418579e-7f;    // 2^-22
constexpr float kAdjFloor = 3.81469727e-6f;  // 2^-18

struct AdjointStop {
    float d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;  // changes of the three previous sweeps

    // Sweep t (1-based) changed mu by at most d, with operands of size s;
    // true when the adjoint ends here.  A NaN (an exchange that timed out)
    // ends it too.
    __device__ __forceinline__ bool done(int t, float d, float s) {
        bool stop = !(d > 0.0f);                             // (a)
        if (!stop && t >= 2) stop = d >= d1 && d <= kAdjFloor * s;  // (c)
        if (!stop && t >= 4) {                               // (b)
            const float rho = fmaxf(fmaxf(d / d1, d1 / d2), d2 / d3);
            stop = rho <= kAdjRhoMax && d * (1.0f + rho) <= kAdjEps * s * (1.0f - rho);
        }
        d3 = d2;
        d2 = d1;
        d1 = d;
        return stop;
    }
};

struct ImpArgs {
    GradSource g;
    const float* P;
    float* r;        // [B,M] sum_k P G
    float* rs;       // [B,M] sum_k P
    float* lam;      // [B,M]
    float* c;        // [B,N] sum_i P G
    float* cs;       // [B,N] sum_i P
    float* mu;       // [B,N]
    float* partA;    // [B,nstrips,N]
    float* partB;    // [B,nstrips,N]
    int nstrips;
    float* grad;     // [B,M,N]
    float* tau_partial;  // [B, gridDim.x]
    float inv_tau;
    int B, M, N, rows;
};

// Row sums of P*G and P, plus their column partials, once per backward: the
// reference recomputes them in every lambda/mu sweep (kernels.cu:986-994,
// :1028-1036).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void imp_prep(ImpArgs a) {
    using R = Row<VEC, CH>;
    extern __shared__ float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int s = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float accA[R::PL], accB[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) accA[e] = accB[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N;
        float p[R::PL], x[R::PL], G[R::PL];
        R::load(a.P + off, lane, a.N, p, 0.0f);
        load_upstream<VEC, CH>(a.g, b, off, lane, a.N, x, G);
        float lr = 0.0f, lrs = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float pg = R::valid(lane, e, a.N) ? p[e] * G[e] : 0.0f;
            lr += pg;
            lrs += p[e];
            accA[e] += pg;
            accB[e] += p[e];
        }
        const float rr = wave_sum(lr);
        const float rrs = wave_sum(lrs);
        if (lane == 0) {
            a.r[bM + i] = rr;
            a.rs[bM + i] = rrs;
            a.lam[bM + i] = 0.0f;  // lambda = mu = 0 before the first sweep (kernels.cu:1712-1713)
        }
    }
    block_column_combine<VEC, CH>(accA, lds, a.N);
    if (wave == 0) R::store(a.partA + (size_t(b) * a.nstrips + s) * a.N, lane, a.N, accA);
    block_column_combine<VEC, CH>(accB, lds, a.N);
    if (wave == 0) R::store(a.partB + (size_t(b) * a.nstrips + s) * a.N, lane, a.N, accB);
}

static __global__ __launch_bounds__(kBlock) void imp_prep_combine(ImpArgs a) {
    const int b = batch_of_block();
    if (b >= a.B) return;
    const float* planes[2] = {a.partA, a.partB};
    float sum[2];
    fold_strips<2>(planes, a.nstrips, a.N, b, sum);
    const int j = fold_col();
    if (fold_lane() != 0 || j >= a.N) return;
    const size_t bj = size_t(b) * a.N + j;
    a.c[bj] = sum[0];
    a.cs[bj] = sum[1];
    a.mu[bj] = 0.0f;
}

// lambda_i = (sum_k P G - sum_k P mu_k) / max(sum_k P, 1e-12)   (kernels.cu:965-1005)
// fused with the column partials sum_i P_ik lambda_i of the mu update.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void imp_lambda_sweep(ImpArgs a) {
    using R = Row<VEC, CH>;
    extern __shared__ float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int s = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float mu[R::PL];
    R::load(a.mu + size_t(b) * a.N, lane, a.N, mu, 0.0f);
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float p[R::PL];
        R::load(a.P + (bM + i) * a.N, lane, a.N, p, 0.0f);
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) d = fmaf(p[e], mu[e], d);
        const float dot = wave_sum(d);
        const float lam = (a.r[bM + i] - dot) / fmaxf(a.rs[bM + i], kSumFloor);
#pragma unroll
        for (int e = 0; e < R::PL; ++e) acc[e] = fmaf(p[e], lam, acc[e]);
        if (lane == 0) a.lam[bM + i] = lam;
    }
    block_column_combine<VEC, CH>(acc, lds, a.N);
    if (wave == 0) R::store(a.partA + (size_t(b) * a.nstrips + s) * a.N, lane, a.N, acc);
}

// mu_k = (sum_i P G - sum_i P lambda_i) / max(sum_i P, 1e-12)   (kernels.cu:1007-1047)
static __global__ __launch_bounds__(kBlock) void imp_mu_combine(ImpArgs a) {
    const int b = batch_of_block();
    if (b >= a.B) return;
    const float* planes[1] = {a.partA};
    float sum[1];
    fold_strips<1>(planes, a.nstrips, a.N, b, sum);
    const int j = fold_col();
    if (fold_lane() != 0 || j >= a.N) return;
    const size_t bj = size_t(b) * a.N + j;
    a.mu[bj] = (a.c[bj] - sum[0]) / fmaxf(a.cs[bj], kSumFloor);
}

// grad = P (G - lambda_i - mu_k) / tau (kernels.cu:1049-1071) with the
// per-block sums of grad * log_alpha for grad_tau (kernels.cu:1073-1098).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void imp_final(ImpArgs a) {
    using R = Row<VEC, CH>;
    __shared__ float scratch[kWavesPerBlock];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = blockIdx.x * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const bool cost_kind = a.g.scores_kind < 0;
    const float gc = a.g.gC ? a.g.gC[b * a.g.gc_step] : 0.0f;
    float mu[R::PL];
    R::load(a.mu + size_t(b) * a.N, lane, a.N, mu, 0.0f);
    float tacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N;
        float p[R::PL], x[R::PL], G[R::PL];
        R::load(a.P + off, lane, a.N, p, 0.0f);
        load_upstream<VEC, CH>(a.g, b, off, lane, a.N, x, G);
        const float lam = a.lam[bM + i];
        float o[R::PL];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float gl = (p[e] * ((G[e] - lam) - mu[e])) * a.inv_tau;
            const float la = cost_kind ? -x[e] : x[e];
            if (R::valid(lane, e, a.N)) tacc = fmaf(gl, la, tacc);
            o[e] = cost_kind ? gc * p[e] - gl : gl - gc * p[e];
        }
        R::store_stream(a.grad + off, lane, a.N, o);
    }
    const float t = block_reduce<kWavesPerBlock>(wave_sum(tacc), scratch, OpSum{});
    if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + blockIdx.x] = t;
}

// -------------------------------------------------------------------------
// Unrolled backward
// -------------------------------------------------------------------------
struct UnrArgs {
    GradSource g;
    float kscale;
    const float* P;
    const float* u_t;      // [B,M] potentials of step t
    const float* v_t;      // [B,N]
    const float* v_tm1;    // [B,N] or null (t = 0: v_{-1} = 0)
    const float* colsum;   // [B,N] column sums of Gamma entering step t
    float* gamma;          // [B,M,N]
    float* partial;        // [B,nstrips,N]
    int nstrips;
    float* grad;           // [B,M,N] written on the final step
    float* tau_partial;    // [B, gridDim.x]
    float inv_tau;
    int B, M, N, rows;
    int final_step;
};

template <int VEC, int CH>
__device__ __forceinline__ void unr_epilogue(const UnrArgs& a, int b, size_t off, int lane,
                                             const float (&gam)[VEC * CH], const float (&p)[VEC * CH],
                                             const float (&x)[VEC * CH], float& tacc) {
    using R = Row<VEC, CH>;
    const bool cost_kind = a.g.scores_kind < 0;
    const float gc = a.g.gC ? a.g.gC[b * a.g.gc_step] : 0.0f;
    float o[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        const float gl = gam[e] * a.inv_tau;               // kernels.cu:926-936
        const float la = cost_kind ? -x[e] : x[e];
        if (R::valid(lane, e, a.N)) tacc = fmaf(gam[e], la, tacc);  // kernels.cu:938-963
        o[e] = cost_kind ? gc * p[e] - gl : gl - gc * p[e];
    }
    R::store_stream(a.grad + off, lane, a.N, o);
}

// Gamma = G * P (kernels.cu:844-854) with its column partial sums; when there
// are no recorded steps it writes the gradient directly.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void unr_init(UnrArgs a) {
    using R = Row<VEC, CH>;
    extern __shared__ float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int s = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    float tacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N;
        float p[R::PL], x[R::PL], G[R::PL];
        R::load(a.P + off, lane, a.N, p, 0.0f);
        load_upstream<VEC, CH>(a.g, b, off, lane, a.N, x, G);
        float gam[R::PL];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            gam[e] = G[e] * p[e];
            acc[e] += gam[e];
        }
        if (a.final_step) unr_epilogue<VEC, CH>(a, b, off, lane, gam, p, x, tacc);
        else R::store(a.gamma + off, lane, a.N, gam);
    }
    if (a.final_step) {
        const float t = block_reduce<kWavesPerBlock>(wave_sum(tacc), lds, OpSum{});
        if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + s] = t;
    } else {
        block_column_combine<VEC, CH>(acc, lds, a.N);
        if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + s) * a.N, lane, a.N, acc);
    }
}

// colsum[b, j] = sum over strips of partial (plain sum, fixed order).
static __global__ __launch_bounds__(kBlock) void column_fold(const float* partial, int nstrips, int B, int N,
                                                     float* out) {
    const int b = batch_of_block();
    if (b >= B) return;
    const float* planes[1] = {partial};
    float sum[1];
    fold_strips<1>(planes, nstrips, N, b, sum);
    const int j = fold_col();
    if (fold_lane() != 0 || j >= N) return;
    out[size_t(b) * N + j] = sum[0];
}

// One reverse step (kernels.cu:1660-1670):
//   Gamma_Y = Gamma - safe_exp(K + u_t + v_t) * colsum(Gamma)
//   Gamma   = Gamma_Y - safe_exp(K + u_t + v_{t-1}) * rowsum(Gamma_Y)
// (safe_exp's clamps on the hardware exponential, safe_fast_exp)
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void unr_step(UnrArgs a) {
    using R = Row<VEC, CH>;
    extern __shared__ float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int s = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const size_t bN = size_t(b) * a.N;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    float tacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N;
        float gam[R::PL], x[R::PL], vec[R::PL];
        R::load(a.gamma + off, lane, a.N, gam, 0.0f);
        R::load(a.g.X + off, lane, a.N, x, 0.0f);
        const float ui = a.u_t[bM + i];
        R::load(a.v_t + bN, lane, a.N, vec, 0.0f);
        float cs[R::PL];
        R::load(a.colsum + bN, lane, a.N, cs, 0.0f);
        float tl = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float ku = x[e] * a.kscale + ui;
            const float q = safe_fast_exp(ku + vec[e]);
            gam[e] = gam[e] - q * cs[e];
            if (R::valid(lane, e, a.N)) tl += gam[e];
        }
        const float ti = wave_sum(tl);
        if (a.v_tm1) R::load(a.v_tm1 + bN, lane, a.N, vec, 0.0f);
        float p[R::PL];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float ku = x[e] * a.kscale + ui;
            const float pe = safe_fast_exp(ku + (a.v_tm1 ? vec[e] : 0.0f));
            gam[e] = gam[e] - pe * ti;
            acc[e] += gam[e];
        }
        if (a.final_step) {
            R::load(a.P + off, lane, a.N, p, 0.0f);
            unr_epilogue<VEC, CH>(a, b, off, lane, gam, p, x, tacc);
        } else {
            R::store(a.gamma + off, lane, a.N, gam);
        }
    }
    if (a.final_step) {
        const float t = block_reduce<kWavesPerBlock>(wave_sum(tacc), lds, OpSum{});
        if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + s] = t;
    } else {
        block_column_combine<VEC, CH>(acc, lds, a.N);
        if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + s) * a.N, lane, a.N, acc);
    }
}

}  // namespace sk
}  // namespace dot_amd
