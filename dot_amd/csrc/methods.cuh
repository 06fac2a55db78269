// Accelerated and scheduled dual Sinkhorn (sinkhorn_dual_forward methods 1-3
// and regularisation schedules, src/sinkhorn/torch_cuda.cpp:61-84, :147-264,
// :323-557).
//
// These methods modify u between the row and the column update (momentum and
// Adam keep a candidate only when it moves closer to the plain update, a
// batch-global test), and Anderson mixes whole (u, v) states, so a row update
// cannot share its exponentials with the next column update as the vanilla
// sweeps do: each iteration is a row-update sweep, a column log-sum-exp
// sweep over row strips (online max/sum per column, strips merged in a fixed
// order) and small vector kernels.  Every decision the reference takes on the
// host after a device-to-host copy (candidate tests, the stop test, Anderson's
// fallback) is a device flag here; iterations after the stop test fired are
// no-ops.  Batch-global maxima of non-negative values go through atomicMax on
// their bit patterns (order-preserving for non-negative floats), so they are
// exact and independent of the order of arrival.
#pragma once

#include <cfloat>
#include <cstdint>

#include "row.cuh"

namespace dot_amd {
namespace mth {

constexpr float kFloor = 1.0e-12f;  // kernels.cu:523-538, :649-664
constexpr int kMaxHistory = 16;     // longest Anderson history (anderson_k) supported

// Natural-log merge of two column states (sum = s * e^m).
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
    const float M = fmaxf(m, m2);
    s = s * expf(m - M) + s2 * expf(m2 - M);
    m = M;
}

__device__ __forceinline__ void atomic_max_nonneg(unsigned* p, float x) {
    atomicMax(p, __float_as_uint(x));
}

// ---------------------------------------------------------------------------
// Row update: u_i = log a_i - (max + log max(sum safe_exp(K_ij + v_j - max), 1e-12)),
// K = X * kscale (kernels.cu:503-545).
// ---------------------------------------------------------------------------
struct RowArgs {
    const float* X;
    float kscale;
    int M, N, rows;
    const float* log_a;  // [B,M] or null
    float log_a_default;
    const float* v;      // [B,N]
    float* u;            // [B,M] out
    const int* done;
};

template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void row_update(RowArgs a) {
    using R = Row<VEC, CH>;
    if (*a.done) return;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = blockIdx.y;
    const int r0 = blockIdx.x * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    float v[R::PL];
    R::load(a.v + size_t(b) * a.N, lane, a.N, v, 0.0f);
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float y[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N, lane, a.N, y, 0.0f);
        float mx = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            y[e] = y[e] * a.kscale + v[e];
            if (R::valid(lane, e, a.N)) mx = fmaxf(mx, y[e]);
        }
        const float m = wave_max(mx);
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, a.N)) s += safe_exp(y[e] - m);
        s = wave_sum(s);
        if (lane == 0) {
            const float la = a.log_a ? a.log_a[size_t(b) * a.M + i] : a.log_a_default;
            a.u[size_t(b) * a.M + i] = la - (m + logf(fmaxf(s, kFloor)));
        }
    }
}

// ---------------------------------------------------------------------------
// Column update: v_j = log b_j - LSE_i(K_ij + u_i) (kernels.cu:629-671), as
// per-strip online (max, sum) states merged in strip order.
// ---------------------------------------------------------------------------
struct ColArgs {
    const float* X;
    float kscale;
    int M, N, rows, nstrips;
    const float* u;      // [B,M]
    float* part_m;       // [B,nstrips,N]
    float* part_s;
    const float* log_b;  // [B,N] or null
    float log_b_default;
    float* v;            // [B,N] out (col_finish)
    const int* done;
};

template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void col_partial(ColArgs a) {
    using R = Row<VEC, CH>;
    extern __shared__ __align__(16) float lds[];  // 2 N floats
    if (*a.done) return;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int st = blockIdx.x;
    const int b = blockIdx.y;
    const int r0 = st * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    float cm[R::PL], cs[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        cm[e] = -FLT_MAX;
        cs[e] = 0.0f;
    }
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float y[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N, lane, a.N, y, 0.0f);
        const float ui = a.u[size_t(b) * a.M + i];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float t = y[e] * a.kscale + ui;
            const float d = t - cm[e];
            const float x = expf(-fabsf(d));
            const bool gt = d > 0.0f;
            cs[e] = gt ? fmaf(cs[e], x, 1.0f) : cs[e] + x;
            cm[e] = gt ? t : cm[e];
        }
    }
    // fold the 4 waves in the order (w0 + w2) + (w1 + w3)
    constexpr int kRounds[3][2] = {{3, 1}, {2, 0}, {1, 0}};
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        __syncthreads();
        if (wave == kRounds[r][0]) {
            R::store(lds, lane, a.N, cm);
            R::store(lds + a.N, lane, a.N, cs);
        }
        __syncthreads();
        if (wave == kRounds[r][1]) {
            float m2[R::PL], s2[R::PL];
            R::load(lds, lane, a.N, m2, -FLT_MAX);
            R::load(lds + a.N, lane, a.N, s2, 0.0f);
#pragma unroll
            for (int e = 0; e < R::PL; ++e) lse_merge(cm[e], cs[e], m2[e], s2[e]);
        }
    }
    if (wave == 0) {
        const size_t off = (size_t(b) * a.nstrips + st) * a.N;
        R::store(a.part_m + off, lane, a.N, cm);
        R::store(a.part_s + off, lane, a.N, cs);
    }
}

constexpr int kFoldCols = 16;
constexpr int kFoldLanes = kBlock / kFoldCols;  // 16

// Strips merged per column: lanes take strips lane, lane + 16, ... in order,
// then a fixed halving tree; v_j = log b_j - (m + log max(s, 1e-12)).
static __global__ __launch_bounds__(kBlock) void col_finish(ColArgs a) {
    __shared__ float sm_m[kFoldLanes][kFoldCols], sm_s[kFoldLanes][kFoldCols];
    if (*a.done) return;
    const int b = blockIdx.y;
    const int jj = threadIdx.x % kFoldCols;
    const int sl = threadIdx.x / kFoldCols;
    const int j = blockIdx.x * kFoldCols + jj;
    float m = -FLT_MAX, s = 0.0f;
    if (j < a.N) {
        const size_t base = size_t(b) * a.nstrips * a.N + j;
        for (int k = sl; k < a.nstrips; k += kFoldLanes)
            lse_merge(m, s, a.part_m[base + size_t(k) * a.N], a.part_s[base + size_t(k) * a.N]);
    }
    sm_m[sl][jj] = m;
    sm_s[sl][jj] = s;
#pragma unroll
    for (int half = kFoldLanes / 2; half >= 1; half /= 2) {
        __syncthreads();
        if (sl < half) {
            lse_merge(m, s, sm_m[sl + half][jj], sm_s[sl + half][jj]);
            sm_m[sl][jj] = m;
            sm_s[sl][jj] = s;
        }
    }
    if (sl == 0 && j < a.N) {
        const float lb = a.log_b ? a.log_b[size_t(b) * a.N + j] : a.log_b_default;
        a.v[size_t(b) * a.N + j] = lb - (m + logf(fmaxf(s, kFloor)));
    }
}

// ---------------------------------------------------------------------------
// Per-iteration flag words (zeroed once per call).  Batch-global maxima of
// non-negative floats are atomicMax over their bit patterns; Anderson's
// minimum |sum(alpha)| is the maximum of kInfBits - bits.
// ---------------------------------------------------------------------------
constexpr int kSlots = 8;
constexpr int kGapU = 0;     // [0] max|cand - target|, [1] max|cur - target| (u step)
constexpr int kGapV = 2;     // the same for the v step
constexpr int kDeltaU = 4;   // stop-test change of u (Anderson: of the state)
constexpr int kDeltaV = 5;   // stop-test change of v
constexpr int kAaMin = 0;    // Anderson: kInfBits - bits(min |sum alpha|)
constexpr int kAaFail = 1;   // Anderson: a solve failed
constexpr unsigned kInfBits = 0x7f800000u;

__device__ __forceinline__ void wave_flag_max(unsigned* p, float x) {
    x = wave_max(x);
    if (threadIdx.x % kWave == 0) atomic_max_nonneg(p, x);
}

static __global__ void reset_counts(int32_t* used, int32_t* converged) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *used = 0;
        *converged = 0;
    }
}

// Momentum candidate (torch_cuda.cpp:470-474): nxt = (1 - omega) cur + omega tgt;
// gaps max|nxt - tgt| -> gap[0], max|cur - tgt| -> gap[1].
static __global__ __launch_bounds__(kBlock) void momentum_candidate(const float* cur, const float* tgt,
                                                                    float* nxt, size_t n, float omega,
                                                                    unsigned* gap, const int* done) {
    // each operation of the reference's tensor expression rounded on its own
#pragma clang fp contract(off)
    if (*done) return;
    float g0 = 0.0f, g1 = 0.0f;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        const float c = cur[i], t = tgt[i];
        const float x = (1.0f - omega) * c + omega * t;
        nxt[i] = x;
        g0 = fmaxf(g0, fabsf(x - t));
        g1 = fmaxf(g1, fabsf(c - t));
    }
    wave_flag_max(gap, g0);
    wave_flag_max(gap + 1, g1);
}

// Adam candidate (torch_cuda.cpp:475-484): the moments always advance; c1, c2
// are the bias-correction divisors (1 when it is off).
static __global__ __launch_bounds__(kBlock) void adam_candidate(const float* cur, const float* tgt, float* nxt,
                                                                float* m1, float* m2, size_t n, float beta1,
                                                                float beta2, float c1, float c2, float lr,
                                                                float eps, unsigned* gap, const int* done) {
#pragma clang fp contract(off)
    if (*done) return;
    float g0 = 0.0f, g1 = 0.0f;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        const float c = cur[i], t = tgt[i];
        const float g = t - c;
        const float mm = beta1 * m1[i] + (1.0f - beta1) * g;
        const float vv = beta2 * m2[i] + (1.0f - beta2) * (g * g);
        m1[i] = mm;
        m2[i] = vv;
        const float x = c + lr * (mm / c1) / (sqrtf(vv / c2) + eps);
        nxt[i] = x;
        g0 = fmaxf(g0, fabsf(x - t));
        g1 = fmaxf(g1, fabsf(c - t));
    }
    wave_flag_max(gap, g0);
    wave_flag_max(gap + 1, g1);
}

// tgt = nxt when the candidate is strictly closer (candidate_improves_cuda,
// torch_cuda.cpp:86-96).
static __global__ __launch_bounds__(kBlock) void accept_candidate(float* tgt, const float* nxt, size_t n,
                                                                  const unsigned* gap, const int* done) {
    if (*done) return;
    if (!(__uint_as_float(gap[0]) < __uint_as_float(gap[1]))) return;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        tgt[i] = nxt[i];
}

// cur = tgt; with `delta` set, max|tgt - cur| -> *delta.
static __global__ __launch_bounds__(kBlock) void commit(float* cur, const float* tgt, size_t n, unsigned* delta,
                                                        const int* done) {
    if (*done) return;
    float d = 0.0f;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        const float t = tgt[i];
        d = fmaxf(d, fabsf(t - cur[i]));
        cur[i] = t;
    }
    if (delta) wave_flag_max(delta, d);
}

// End of iteration `it` (slots of that iteration): count it, and stop when
// tol > 0 and the larger of the two deltas is below tol.
static __global__ void finish_iteration(const unsigned* slots, int it, float tol, int* done, int32_t* used,
                                        int32_t* converged) {
    if (blockIdx.x != 0 || threadIdx.x != 0 || *done) return;
    *used = it + 1;
    const float d = fmaxf(__uint_as_float(slots[kDeltaU]), __uint_as_float(slots[kDeltaV]));
    if (tol > 0.0f && d < tol) {
        *converged = 1;
        *done = 1;
    }
}

// ---------------------------------------------------------------------------
// Anderson mixing (torch_cuda.cpp:395-446) on the state x = (u, v) of each
// batch element, with a ring of up to kMaxHistory (x, f = x_new - x) pairs.
// ---------------------------------------------------------------------------
struct AaArgs {
    int B, M, N;
    float* xu;        // [B,M] state
    float* xv;        // [B,N]
    const float* nu;  // [B,M] x_new
    const float* nv;  // [B,N]
    float* hxu;       // [k,B,M] states
    float* hxv;       // [k,B,N]
    float* hfu;       // [k,B,M] residuals
    float* hfv;       // [k,B,N]
    int slot;         // physical slot of the newest pair
    int h;            // pairs held after the push
    int order[kMaxHistory];  // physical slots, oldest first
    float mixing_beta;
    float* gram;      // [B,kMaxHistory,kMaxHistory]
    float* alpha;     // [B,kMaxHistory]
    float* denom;     // [B]
    unsigned* slots;  // this iteration's flag words
    int track_delta;
    const int* done;
};

__device__ __forceinline__ float aa_at(const float* hu, const float* hv, int s, size_t nu, size_t nv, int b, int M,
                                       int N, int i) {
    return i < M ? hu[size_t(s) * nu + size_t(b) * M + i] : hv[size_t(s) * nv + size_t(b) * N + (i - M)];
}

// Push (x, x_new - x) into the ring; the residual's max into the delta slot.
static __global__ __launch_bounds__(kBlock) void aa_push(AaArgs a) {
    if (*a.done) return;
    const size_t nu = size_t(a.B) * a.M, nv = size_t(a.B) * a.N, n = nu + nv;
    float d = 0.0f;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        if (i < nu) {
            const float x = a.xu[i], f = a.nu[i] - x;
            a.hxu[size_t(a.slot) * nu + i] = x;
            a.hfu[size_t(a.slot) * nu + i] = f;
            d = fmaxf(d, fabsf(f));
        } else {
            const size_t k = i - nu;
            const float x = a.xv[k], f = a.nv[k] - x;
            a.hxv[size_t(a.slot) * nv + k] = x;
            a.hfv[size_t(a.slot) * nv + k] = f;
            d = fmaxf(d, fabsf(f));
        }
    }
    if (a.track_delta) wave_flag_max(a.slots + kDeltaU, d);
}

// Row p of the Gram matrix F^T F of element b (grid h x B): one pass over the
// element's M + N residual entries of every history pair.
static __global__ __launch_bounds__(kBlock) void aa_gram(AaArgs a) {
    __shared__ float red[kWavesPerBlock][kMaxHistory];
    if (*a.done) return;
    const int p = blockIdx.x, b = blockIdx.y, h = a.h;
    const size_t nu = size_t(a.B) * a.M, nv = size_t(a.B) * a.N;
    const int sp = a.order[p];
    float acc[kMaxHistory];
#pragma unroll
    for (int q = 0; q < kMaxHistory; ++q) acc[q] = 0.0f;
    for (int i = threadIdx.x; i < a.M + a.N; i += kBlock) {
        const float fp = aa_at(a.hfu, a.hfv, sp, nu, nv, b, a.M, a.N, i);
#pragma unroll
        for (int q = 0; q < kMaxHistory; ++q)
            if (q < h) acc[q] = fmaf(fp, aa_at(a.hfu, a.hfv, a.order[q], nu, nv, b, a.M, a.N, i), acc[q]);
    }
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
    for (int q = 0; q < kMaxHistory; ++q) {
        const float s = wave_sum(acc[q]);
        if (lane == 0) red[wave][q] = s;
    }
    __syncthreads();
    if (threadIdx.x < h) {
        const int q = threadIdx.x;
        float s = red[0][q];
#pragma unroll
        for (int w = 1; w < kWavesPerBlock; ++w) s += red[w][q];
        a.gram[(size_t(b) * kMaxHistory + p) * kMaxHistory + q] = s;
    }
}

// (G + 1e-8 I) alpha = 1 for element b by Gaussian elimination with partial
// pivoting (one thread; h <= kMaxHistory), then sum(alpha); a zero or
// non-finite pivot or sum marks the iteration's solve as failed.
static __global__ void aa_solve(AaArgs a) {
    __shared__ float A[kMaxHistory][kMaxHistory + 1];
    __shared__ float x[kMaxHistory];
    if (*a.done || threadIdx.x != 0) return;
    const int b = blockIdx.x, h = a.h;
    for (int p = 0; p < h; ++p) {
        for (int q = 0; q < h; ++q)
            A[p][q] = a.gram[(size_t(b) * kMaxHistory + p) * kMaxHistory + q] + (p == q ? 1.0e-8f : 0.0f);
        x[p] = 1.0f;
    }
    bool failed = false;
    for (int c = 0; c < h && !failed; ++c) {
        int piv = c;
        for (int r = c + 1; r < h; ++r)
            if (fabsf(A[r][c]) > fabsf(A[piv][c])) piv = r;
        const float pv = A[piv][c];
        if (pv == 0.0f || !(fabsf(pv) <= FLT_MAX)) {
            failed = true;
            break;
        }
        if (piv != c) {
            for (int q = 0; q < h; ++q) {
                const float t = A[c][q];
                A[c][q] = A[piv][q];
                A[piv][q] = t;
            }
            const float t = x[c];
            x[c] = x[piv];
            x[piv] = t;
        }
        for (int r = c + 1; r < h; ++r) {
            const float f = A[r][c] / A[c][c];
            for (int q = c; q < h; ++q) A[r][q] -= f * A[c][q];
            x[r] -= f * x[c];
        }
    }
    float sum = 0.0f;
    if (!failed) {
        for (int c = h - 1; c >= 0; --c) {
            float t = x[c];
            for (int q = c + 1; q < h; ++q) t -= A[c][q] * x[q];
            x[c] = t / A[c][c];
        }
        for (int c = 0; c < h; ++c) sum += x[c];
        failed = !(fabsf(sum) <= FLT_MAX);
    }
    for (int c = 0; c < h; ++c) a.alpha[size_t(b) * kMaxHistory + c] = failed ? 0.0f : x[c];
    a.denom[b] = sum;
    if (failed) atomicOr(a.slots + kAaFail, 1u);
    else atomicMax(a.slots + kAaMin, kInfBits - __float_as_uint(fabsf(sum)));
}

// x = sum_c (alpha_c / sum) (X_c + beta F_c) when every element's solve
// succeeded with |sum| >= 1e-12, else x = x_new (torch_cuda.cpp:421-444).
// With fewer than two pairs, x = x_new.
static __global__ __launch_bounds__(kBlock) void aa_update(AaArgs a) {
    if (*a.done) return;
    const bool mix = a.h >= 2 && a.slots[kAaFail] == 0u &&
                     __uint_as_float(kInfBits - a.slots[kAaMin]) >= 1.0e-12f;
    const size_t nu = size_t(a.B) * a.M, nv = size_t(a.B) * a.N, n = nu + nv;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        const bool isu = i < nu;
        const size_t k = isu ? i : i - nu;
        float x;
        if (!mix) {
            x = isu ? a.nu[k] : a.nv[k];
        } else {
            const int b = int(isu ? k / size_t(a.M) : k / size_t(a.N));
            const float den = a.denom[b];
            const float* hx = isu ? a.hxu : a.hxv;
            const float* hf = isu ? a.hfu : a.hfv;
            const size_t stride = isu ? nu : nv;
            x = 0.0f;
#pragma unroll
            for (int c = 0; c < kMaxHistory; ++c) {
                if (c < a.h) {
                    const float al = a.alpha[size_t(b) * kMaxHistory + c] / den;
                    const size_t off = size_t(a.order[c]) * stride + k;
                    x = fmaf(hx[off] + a.mixing_beta * hf[off], al, x);
                }
            }
        }
        if (isu) a.xu[k] = x;
        else a.xv[k] = x;
    }
}

// ---------------------------------------------------------------------------
// Plan: exp(K + u_i + v_j) (or its log) with K at the target tau, and the
// per-strip share of sum(P C), C = csign * X (torch_cuda.cpp:550-552).
// ---------------------------------------------------------------------------
struct PlanArgs {
    const float* X;
    float kscale, csign;
    int M, N, rows, return_log;
    int safe;             // safe_exp (the vanilla materialisation) rather than exp
    const float* u;
    const float* v;
    float* plan;          // or null
    float* cost_partial;  // [B,nstrips] or null
};

template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void plan(PlanArgs a) {
    using R = Row<VEC, CH>;
    __shared__ float scratch[kWavesPerBlock];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = blockIdx.y;
    const int r0 = blockIdx.x * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    float v[R::PL];
    R::load(a.v + size_t(b) * a.N, lane, a.N, v, 0.0f);
    float cacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (size_t(b) * a.M + i) * a.N;
        float x[R::PL];
        R::load(a.X + off, lane, a.N, x, 0.0f);
        const float ui = a.u[size_t(b) * a.M + i];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float lp = x[e] * a.kscale + ui + v[e];
            const float p = a.return_log ? lp : (a.safe ? safe_exp(lp) : expf(lp));
            if (a.cost_partial && R::valid(lane, e, a.N)) cacc = fmaf(p, a.csign * x[e], cacc);
            x[e] = p;
        }
        if (a.plan) R::store(a.plan + off, lane, a.N, x);
    }
    if (a.cost_partial) {
        const float s = block_reduce<kWavesPerBlock>(wave_sum(cacc), scratch, OpSum{});
        if (threadIdx.x == 0) a.cost_partial[size_t(b) * gridDim.x + blockIdx.x] = s;
    }
}

}  // namespace mth
}  // namespace dot_amd
