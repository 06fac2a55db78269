// Accelerated and scheduled dual Sinkhorn (sinkhorn_dual_forward methods 1-3
// and regularisation schedules, src/sinkhorn/torch_cuda.cpp:61-84, :147-264,
// :323-557).
//
// One iteration is one pass over the matrix (sweep) and a per-column kernel
// (vfinish):
//   sweep     row update u*_i = log a_i - LSE_j(K_ij + v_j) for a strip of rows,
//             the method's candidate u'_i (momentum: (1 - w) u + w u*;
//             Adam: moment-scaled step), and per-strip column sums of
//             exp(K_ij + u_i + v_j) for BOTH u = u* and u = u': they share the
//             row's exponentials, e_ij w_i and e_ij w_i exp(u'_i - u*_i), so
//             keeping either candidate costs no second pass;
//   vfinish   the column update from whichever sum the batch-global test kept
//             (v*_j = log b_j + v_j - log colsum_j), the v candidate, and its test.
// The reference decides each test on the host after a device-to-host copy;
// here every decision is a word of the iteration's flag block, read by the
// kernels that need it: the sweep of iteration t takes the u and v that
// iteration t-1 kept, and returns at once when iteration t-1 met the stop
// test.  An iteration that did not run leaves its flag words zero, which
// reads as met, so the stop carries forward with no extra state.  Anderson
// runs the plain sweep and mixes the (u, v) state with small vector kernels.
// Batch-global maxima of non-negative values are atomicMax over their bit
// patterns (order-preserving for non-negative floats): exact and independent
// of the order of arrival.
#pragma once

#include <cfloat>
#include <cstdint>

#include "row.cuh"
#include "tile.cuh"

namespace dot_amd {
namespace mth {

constexpr float kSumFloor = 1.0e-12f;     // log(max(sum, 1e-12)), kernels.cu:523-538, :649-664
constexpr float kColSumFloor = 1.0e-20f;  // smaller column sums take the exact column LSE
constexpr int kMaxHistory = 64;           // longest Anderson ring held (pairs)

// Solver codes (the reference's method codes); Anderson runs the plain sweep.
constexpr int kPlain = 0, kMomentum = 1, kAnderson = 2, kAdam = 3;

// Flag words of one iteration (zeroed once per call).  Each word is striped
// over kStripes addresses: a workgroup reduces its values first and adds them
// with one atomicMax on the stripe of its index, so no address sees more than
// a few dozen atomics per launch; readers take the max over the stripes with
// one wave-wide load.
constexpr int kStripes = kWave;
constexpr int kGapU = 0;    // [0] max|u' - u*|, [1] max|u - u*| (the change when u* is kept)
constexpr int kGapV = 2;    // the same for v
constexpr int kMoveU = 4;   // max|u' - u| (the change when u' is kept)
constexpr int kMoveV = 5;
constexpr int kAaDelta = 6; // Anderson: max|x_new - x|
constexpr int kAaMin = 7;   // Anderson: kInfBits - bits(min |sum alpha|), ordered as a float
constexpr int kAaFail = 8;  // Anderson: a solve failed
constexpr int kWords = 9;
constexpr int kIterWords = kWords * kStripes;
// a word's stripes are contiguous, so a wave reads one word in one access
__host__ __device__ constexpr int flag_at(int k, int stripe) { return k * kStripes + stripe; }
constexpr unsigned kInfBits = 0x7f800000u;

// Word k of an iteration's flag block; every lane of the wave must call it.
__device__ __forceinline__ float flag(const unsigned* s, int k) {
    return wave_max(__uint_as_float(s[flag_at(k, threadIdx.x % kWave)]));
}

inline float host_flag(const unsigned* s, int k) {
    float m = 0.0f;
    for (int i = 0; i < kStripes; ++i) {
        const float x = __builtin_bit_cast(float, s[flag_at(k, i)]);
        m = x > m ? x : m;
    }
    return m;
}

// What an iteration decided: candidate tests (candidate_improves_cuda,
// torch_cuda.cpp:86-96) and the stop test's change (torch_cuda.cpp:230-238
// vanilla, u only; :519-524 momentum/Adam, u and v after the tests; :400
// Anderson).  An iteration that did not run reads as all zero.
struct Decision {
    bool keep_u, keep_v;
    float delta;
};

template <class Flag>
__host__ __device__ inline Decision decide(Flag f, int method) {
    Decision d{false, false, 0.0f};
    if (method == kAnderson) {
        d.delta = f(kAaDelta);
        return d;
    }
    const float g1 = f(kGapU + 1);
    if (method == kPlain) {
        d.delta = g1;
        return d;
    }
    d.keep_u = f(kGapU) < g1;
    const float h1 = f(kGapV + 1);
    d.keep_v = f(kGapV) < h1;
    const float du = d.keep_u ? f(kMoveU) : g1;
    const float dv = d.keep_v ? f(kMoveV) : h1;
    d.delta = du > dv ? du : dv;
    return d;
}

// This lane's stripe of every word of a flag block (zeros for null), so the
// loads can be issued together with a kernel's other operands.
struct Words {
    float w[kWords];
};

__device__ __forceinline__ Words load_words(const unsigned* s) {
    const int lane = threadIdx.x % kWave;
    Words r;
#pragma unroll
    for (int k = 0; k < kWords; ++k) r.w[k] = s ? __uint_as_float(s[flag_at(k, lane)]) : 0.0f;
    return r;
}

// The decision from loaded words.  Every lane of the wave must call it.
__device__ __forceinline__ Decision decide_words(Words r, int method) {
#pragma unroll
    for (int k = 0; k < kWords; ++k) r.w[k] = wave_max(r.w[k]);
    return decide([&](int k) { return r.w[k]; }, method);
}

__device__ __forceinline__ Decision decide_dev(const unsigned* s, int method) {
    return decide_words(load_words(s), method);
}

inline Decision decide_host(const unsigned* s, int method) {
    return decide([&](int k) { return host_flag(s, k); }, method);
}

// The previous iteration's decision (prev null before the first) and whether
// the stop test fired at or before it.  Every lane of the wave must call it.
struct Prev {
    Decision d;
    bool stop;
};

__device__ __forceinline__ Prev previous_from(const Words& w, bool has_prev, int method, float tol) {
    Prev p{{false, false, 0.0f}, false};
    if (has_prev) {
        p.d = decide_words(w, method);
        p.stop = tol > 0.0f && p.d.delta < tol;
    }
    return p;
}

__device__ __forceinline__ Prev previous(const unsigned* prev, int method, float tol) {
    return previous_from(load_words(prev), prev != nullptr, method, tol);
}

__device__ __forceinline__ void atomic_max_nonneg(unsigned* p, float x) { atomicMax(p, __float_as_uint(x)); }

// Workgroup maxima of up to three values per thread, each added to its word's
// stripe for this workgroup by its own thread (one barrier for all).  Every
// thread must call it; `red` holds 3 * kWavesPerBlock floats that no other
// code of the kernel uses.  Words are scalars (an index array would be
// placed in scratch memory and indexed there).
template <int NW>
__device__ __forceinline__ void block_flag_max(unsigned* s, int k0, float x0, int k1, float x1, int k2, float x2,
                                               float* red) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const float m0 = wave_max(x0);
    const float m1 = NW > 1 ? wave_max(x1) : 0.0f;
    const float m2 = NW > 2 ? wave_max(x2) : 0.0f;
    if (lane == 0) {
        red[wave] = m0;
        if (NW > 1) red[kWavesPerBlock + wave] = m1;
        if (NW > 2) red[2 * kWavesPerBlock + wave] = m2;
    }
    __syncthreads();
    if (threadIdx.x < NW) {
        const int w = threadIdx.x;
        float m = red[w * kWavesPerBlock];
#pragma unroll
        for (int i = 1; i < kWavesPerBlock; ++i) m = fmaxf(m, red[w * kWavesPerBlock + i]);
        const int k = w == 0 ? k0 : (w == 1 ? k1 : k2);
        const unsigned blk = blockIdx.x + blockIdx.y * gridDim.x;
        atomic_max_nonneg(s + flag_at(k, blk % kStripes), m);
    }
}

// ---------------------------------------------------------------------------
// Sweep
// ---------------------------------------------------------------------------
struct SweepArgs {
    const float* X;
    float kscale;               // K = X * kscale at this iteration's tau
    int B, M, N, rows, nstrips;
    const float* log_a;         // [B,M] or null
    float log_a_default;
    const float* u_prev[2];     // [B,M] u* and u' of the previous iteration (null: zeros)
    const float* v_prev[2];     // [B,N]
    const unsigned* prev;       // flag words of the previous iteration, null at the first
    unsigned* slots;            // this iteration's
    int method;                 // for the stop test
    float tol;
    int track;                  // write the change words (tol > 0)
    float* ut;                  // [B,M] out: u*
    float* un;                  // [B,M] out: u'
    float* m1;                  // [B,M] Adam moments (in place)
    float* m2;
    float omega, lr, beta1, beta2, c1, c2, eps;
    float* part_t;              // [B,nstrips,N] column sums with u*
    float* part_n;              // [B,nstrips,N] column sums with u'
    int t;                      // iteration
    int32_t* used;              // iterations executed (written by every sweep that runs)
    int32_t* converged;         // set by the first sweep that finds the stop test met
};

template <int VEC, int CH, int MODE>
__global__ __launch_bounds__(kBlock) void sweep(SweepArgs a) {
    // the candidates round each operation of the reference's tensor
    // expressions on its own; the row arithmetic uses explicit fmaf
#pragma clang fp contract(off)
    using R = Row<VEC, CH>;
    extern __shared__ __align__(16) float lds[];  // 2 N floats + 3 kWavesPerBlock
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int s = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    // the previous iteration's flags and both of its v candidates, loaded
    // together before anything waits on them
    const Words words = load_words(a.prev);
    float v[R::PL], v_alt[R::PL];
    if (a.v_prev[0]) {
        R::load(a.v_prev[0] + size_t(b) * a.N, lane, a.N, v, 0.0f);
        if constexpr (MODE != kPlain) R::load(a.v_prev[1] + size_t(b) * a.N, lane, a.N, v_alt, 0.0f);
    } else {
#pragma unroll
        for (int e = 0; e < R::PL; ++e) v[e] = v_alt[e] = 0.0f;
    }
    const Prev pv = previous_from(words, a.prev != nullptr, a.method, a.tol);
    const bool first_block = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0;
    if (pv.stop) {
        if (first_block) *a.converged = 1;
        return;
    }
    if (first_block) *a.used = a.t + 1;
    if constexpr (MODE != kPlain) {
        if (pv.d.keep_v)
#pragma unroll
            for (int e = 0; e < R::PL; ++e) v[e] = v_alt[e];
    }
    const int r0 = s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    // static indices only: a dynamic index into the kernel-argument array
    // would copy it to scratch
    const float* uc = MODE != kPlain && pv.d.keep_u ? a.u_prev[1] : a.u_prev[0];
    float acc_t[R::PL], acc_n[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc_t[e] = acc_n[e] = 0.0f;
    float gap0 = 0.0f, gap1 = 0.0f, move = 0.0f;

    auto row = [&](int i, RowBuf<R>& buf) {
        float(&x)[R::PL] = buf.v;
        float mloc = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] = R::valid(lane, e, a.N) ? fmaf(x[e], a.kscale, v[e]) : -INFINITY;
            mloc = fmaxf(mloc, x[e]);
        }
        const float m = wave_max(mloc);
        float sloc = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] = fast_exp(x[e] - m);
            sloc += x[e];
        }
        const float ssum = wave_sum(sloc);
        const float lga = a.log_a ? a.log_a[bM + i] : a.log_a_default;
        const float ls = logf(fmaxf(ssum, kSumFloor));
        const float ut = lga - (m + ls);
        const float w = fast_exp(lga - ls);  // e_ij w = exp(K_ij + v_j + u*_i)
#pragma unroll
        for (int e = 0; e < R::PL; ++e) acc_t[e] = fmaf(x[e], w, acc_t[e]);
        const float ucur = uc ? uc[bM + i] : 0.0f;
        if constexpr (MODE == kPlain) {
            gap1 = fmaxf(gap1, fabsf(ucur - ut));
            if (lane == 0) a.ut[bM + i] = ut;
        } else {
            float un;
            if constexpr (MODE == kMomentum) {
                un = (1.0f - a.omega) * ucur + a.omega * ut;  // torch_cuda.cpp:470-474
            } else {
                // torch_cuda.cpp:475-484: the moments advance whether or not u' is kept
                const float g = ut - ucur;
                const float mm = a.beta1 * a.m1[bM + i] + (1.0f - a.beta1) * g;
                const float vv = a.beta2 * a.m2[bM + i] + (1.0f - a.beta2) * (g * g);
                if (lane == 0) {
                    a.m1[bM + i] = mm;
                    a.m2[bM + i] = vv;
                }
                un = ucur + a.lr * (mm / a.c1) / (sqrtf(vv / a.c2) + a.eps);
            }
            const float w2 = w * fast_exp(un - ut);  // e_ij w2 = exp(K_ij + v_j + u'_i)
#pragma unroll
            for (int e = 0; e < R::PL; ++e) acc_n[e] = fmaf(x[e], w2, acc_n[e]);
            gap0 = fmaxf(gap0, fabsf(un - ut));
            gap1 = fmaxf(gap1, fabsf(ucur - ut));
            move = fmaxf(move, fabsf(un - ucur));
            if (lane == 0) {
                a.ut[bM + i] = ut;
                a.un[bM + i] = un;
            }
        }
    };
    auto load = [&](int i, RowBuf<R>& buf) { R::load_clamped(a.X + (bM + i) * a.N, lane, a.N, buf.v, 0.0f); };
    if constexpr (R::PL <= 16) {
        // short rows: each row's load is issued one row ahead (rows of 32
        // floats per lane would need the second buffer's registers)
        pipelined_rows<RowBuf<R>>(r0 + wave, r1, kWavesPerBlock, load, row);
    } else {
        for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
            RowBuf<R> buf;
            load(i, buf);
            row(i, buf);
        }
    }

    const size_t off = (size_t(b) * a.nstrips + s) * a.N;
    block_column_combine<VEC, CH>(acc_t, lds, a.N);
    if (wave == 0) R::store(a.part_t + off, lane, a.N, acc_t);
    if constexpr (MODE != kPlain) {
        block_column_combine<VEC, CH>(acc_n, lds, a.N);
        if (wave == 0) R::store(a.part_n + off, lane, a.N, acc_n);
    }
    // every lane holds its wave's maxima (wave-uniform values)
    float* red = lds + 2 * a.N;
    if constexpr (MODE != kPlain) {
        block_flag_max<3>(a.slots, kGapU, gap0, kGapU + 1, gap1, kMoveU, move, red);
    } else if (a.track) {
        block_flag_max<1>(a.slots, kGapU + 1, gap1, 0, 0.0f, 0, 0.0f, red);
    }
}

// ---------------------------------------------------------------------------
// The sweep for rows longer than kMaxRowLen, in three launches over the
// strips x chunks tiling of tile.cuh (workgroup (s, c) owns rows
// [s*rows, (s+1)*rows) and columns [c*kChunk, (c+1)*kChunk)):
//   wide_rows    per row and chunk, (max, sum) of exp over K_ij + v_j;
//   wide_finish  per row, the chunk partials folded in chunk order into u*,
//                the method's candidate u' (Adam's moments advanced once),
//                the flag maxima, and the row's shift m_i and weights
//                w_i = a_i / s_i, w2_i = w_i exp(u'_i - u*_i);
//   wide_cols    per tile, the column sums sum_i exp(K_ij + v_j - m_i) w_i
//                (and w2_i) of the chunk's columns, one partial row per strip
//                in the [B, nstrips, N] layout vfinish reads.
// The values are those of the fused sweep up to the rounding of the chunked
// log-sum-exp.
// ---------------------------------------------------------------------------
struct WideArgs {
    SweepArgs s;       // nstrips counts strips of the tiling; rows is its strip height
    int nchunks;
    float2* rpart;     // [B, nchunks, M] chunk (max, sum)
    float* row_m;      // [B, M] the row's max of K + v
    float* row_w;      // [B, M] a_i / s_i
    float* row_w2;     // [B, M] (a_i / s_i) exp(u'_i - u*_i)
};

// The previous iteration's decision and the v this iteration sweeps with
// (v* or v', chunk columns); false when the stop test fired before it.
template <class R, int MODE>
__device__ __forceinline__ bool wide_prologue(const SweepArgs& a, int b, int c0, int nc, Prev& pv,
                                              float (&v)[R::PL]) {
    const int lane = threadIdx.x % kWave;
    const Words words = load_words(a.prev);
    float v_alt[R::PL];
    if (a.v_prev[0]) {
        R::load(a.v_prev[0] + size_t(b) * a.N + c0, lane, nc, v, 0.0f);
        if constexpr (MODE != kPlain) R::load(a.v_prev[1] + size_t(b) * a.N + c0, lane, nc, v_alt, 0.0f);
    } else {
#pragma unroll
        for (int e = 0; e < R::PL; ++e) v[e] = v_alt[e] = 0.0f;
    }
    pv = previous_from(words, a.prev != nullptr, a.method, a.tol);
    if (pv.stop) return false;
    if constexpr (MODE != kPlain) {
        if (pv.d.keep_v)
#pragma unroll
            for (int e = 0; e < R::PL; ++e) v[e] = v_alt[e];
    }
    return true;
}

template <int VEC, int CH, int MODE>
__global__ __launch_bounds__(kBlock) void wide_rows(WideArgs w) {
#pragma clang fp contract(off)
    using R = Row<VEC, CH>;
    const SweepArgs& a = w.s;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const wide::Tile tl = wide::tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    Prev pv;
    float v[R::PL];
    if (!wide_prologue<R, MODE>(a, b, tl.c0, tl.nc, pv, v)) return;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float2* part = w.rpart + (size_t(b) * w.nchunks + tl.c) * a.M;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (bM + i) * a.N + tl.c0, lane, tl.nc, x, 0.0f);
        float mloc = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] = R::valid(lane, e, tl.nc) ? fmaf(x[e], a.kscale, v[e]) : -INFINITY;
            mloc = fmaxf(mloc, x[e]);
        }
        const float m = wave_max(mloc);
        float sloc = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) sloc += fast_exp(x[e] - m);
        const float s = wave_sum(sloc);
        if (lane == 0) part[i] = make_float2(m, s);
    }
}

constexpr int kFinishRowsPerWave = 8;

template <int MODE>
__global__ __launch_bounds__(kBlock) void wide_finish(WideArgs w) {
#pragma clang fp contract(off)
    const SweepArgs& a = w.s;
    __shared__ float red[3 * kWavesPerBlock];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const Prev pv = previous(a.prev, a.method, a.tol);
    const bool first_block = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0;
    if (pv.stop) {
        if (first_block) *a.converged = 1;
        return;
    }
    if (first_block) *a.used = a.t + 1;
    const float* uc = MODE != kPlain && pv.d.keep_u ? a.u_prev[1] : a.u_prev[0];
    const size_t bM = size_t(b) * a.M;
    const float2* part = w.rpart + size_t(b) * w.nchunks * a.M;
    const int i0 = (blockIdx.x * kWavesPerBlock + wave) * kFinishRowsPerWave;
    const int i1 = min(i0 + kFinishRowsPerWave, a.M);
    float gap0 = 0.0f, gap1 = 0.0f, move = 0.0f;
    for (int i = i0; i < i1; ++i) {
        float m, ssum;
        wide::fold_lse(part + i, a.M, w.nchunks, m, ssum);
        const float lga = a.log_a ? a.log_a[bM + i] : a.log_a_default;
        const float ls = logf(fmaxf(ssum, kSumFloor));
        const float ut = lga - (m + ls);
        const float wt = fast_exp(lga - ls);
        const float ucur = uc ? uc[bM + i] : 0.0f;
        float un = ut;
        if constexpr (MODE == kPlain) {
            gap1 = fmaxf(gap1, fabsf(ucur - ut));
        } else {
            if constexpr (MODE == kMomentum) {
                un = (1.0f - a.omega) * ucur + a.omega * ut;  // torch_cuda.cpp:470-474
            } else {
                // torch_cuda.cpp:475-484: the moments advance whether or not u' is kept
                const float g = ut - ucur;
                const float mm = a.beta1 * a.m1[bM + i] + (1.0f - a.beta1) * g;
                const float vv = a.beta2 * a.m2[bM + i] + (1.0f - a.beta2) * (g * g);
                if (lane == 0) {
                    a.m1[bM + i] = mm;
                    a.m2[bM + i] = vv;
                }
                un = ucur + a.lr * (mm / a.c1) / (sqrtf(vv / a.c2) + a.eps);
            }
            gap0 = fmaxf(gap0, fabsf(un - ut));
            gap1 = fmaxf(gap1, fabsf(ucur - ut));
            move = fmaxf(move, fabsf(un - ucur));
        }
        if (lane == 0) {
            a.ut[bM + i] = ut;
            if constexpr (MODE != kPlain) {
                a.un[bM + i] = un;
                w.row_w2[bM + i] = wt * fast_exp(un - ut);
            }
            w.row_m[bM + i] = m;
            w.row_w[bM + i] = wt;
        }
    }
    if constexpr (MODE != kPlain) {
        block_flag_max<3>(a.slots, kGapU, gap0, kGapU + 1, gap1, kMoveU, move, red);
    } else if (a.track) {
        block_flag_max<1>(a.slots, kGapU + 1, gap1, 0, 0.0f, 0, 0.0f, red);
    }
}

template <int VEC, int CH, int MODE>
__global__ __launch_bounds__(kBlock) void wide_cols(WideArgs w) {
#pragma clang fp contract(off)
    using R = Row<VEC, CH>;
    const SweepArgs& a = w.s;
    extern __shared__ __align__(16) float lds[];  // 2 kChunk floats
    const int b = batch_of_block();
    if (b >= a.B) return;
    const wide::Tile tl = wide::tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    Prev pv;
    float v[R::PL];
    if (!wide_prologue<R, MODE>(a, b, tl.c0, tl.nc, pv, v)) return;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float acc_t[R::PL], acc_n[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc_t[e] = acc_n[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (bM + i) * a.N + tl.c0, lane, tl.nc, x, 0.0f);
        const float m = w.row_m[bM + i];
        const float wt = w.row_w[bM + i];
        const float w2 = MODE != kPlain ? w.row_w2[bM + i] : 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float y = R::valid(lane, e, tl.nc) ? fmaf(x[e], a.kscale, v[e]) : -INFINITY;
            const float ex = fast_exp(y - m);
            acc_t[e] = fmaf(ex, wt, acc_t[e]);
            if constexpr (MODE != kPlain) acc_n[e] = fmaf(ex, w2, acc_n[e]);
        }
    }
    const size_t off = (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0;
    block_column_combine<VEC, CH>(acc_t, lds, tl.nc);
    if (wave == 0) R::store(a.part_t + off, lane, tl.nc, acc_t);
    if constexpr (MODE != kPlain) {
        block_column_combine<VEC, CH>(acc_n, lds, tl.nc);
        if (wave == 0) R::store(a.part_n + off, lane, tl.nc, acc_n);
    }
}

// ---------------------------------------------------------------------------
// Column update and the v candidate: 64 columns per workgroup, 4 threads per
// column summing its strips (lane-strided, then a fixed halving tree).  Wider
// workgroups mean fewer of them, and so fewer flag atomics and barriers: with
// 16 columns per workgroup the momentum iteration took 6 µs longer.
// ---------------------------------------------------------------------------
struct VfinishArgs {
    const float* X;
    float kscale;
    int B, M, N, nstrips;
    const float* log_b;         // [B,N] or null
    float log_b_default;
    const float* v_prev[2];     // as SweepArgs
    const float* ut;            // [B,M] this iteration's u* and u' (exact fallback)
    const float* un;
    const unsigned* prev;
    unsigned* slots;            // this iteration's (the u test decided by the sweep)
    int method;
    float tol;
    const float* part_t;
    const float* part_n;
    float* vt;                  // [B,N] out: v*
    float* vn;                  // [B,N] out: v'
    float* m1;                  // [B,N] Adam moments
    float* m2;
    float omega, lr, beta1, beta2, c1, c2, eps;
};

constexpr int kFoldCols = 64;
constexpr int kFoldLanes = kBlock / kFoldCols;  // 4 threads per column

template <int MODE>
__global__ __launch_bounds__(kBlock) void vfinish(VfinishArgs a) {
#pragma clang fp contract(off)
    __shared__ float fold[kFoldLanes][kFoldCols];
    __shared__ float red[3 * kWavesPerBlock];
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int jj = threadIdx.x % kFoldCols;
    const int sl = threadIdx.x / kFoldCols;
    const int j = blockIdx.x * kFoldCols + jj;
    const int lane = threadIdx.x % kWave;
    // every operand is loaded before the decisions that select among them
    const Words words = load_words(a.prev);
    float g0 = 0.0f, g1 = 0.0f;
    if constexpr (MODE != kPlain) {
        g0 = __uint_as_float(a.slots[flag_at(kGapU, lane)]);
        g1 = __uint_as_float(a.slots[flag_at(kGapU + 1, lane)]);
    }
    float cs_t = 0.0f, cs_n = 0.0f;
    if (j < a.N) {
        const size_t off = size_t(b) * a.nstrips * a.N + j;
        for (int s = sl; s < a.nstrips; s += kFoldLanes) {
            cs_t += a.part_t[off + size_t(s) * a.N];
            if constexpr (MODE != kPlain) cs_n += a.part_n[off + size_t(s) * a.N];
        }
    }
    const bool col = sl == 0 && j < a.N;
    const size_t bj = size_t(b) * a.N + j;
    float lgb = a.log_b_default, v0 = 0.0f, v1 = 0.0f, m1 = 0.0f, m2 = 0.0f;
    if (col) {
        if (a.log_b) lgb = a.log_b[bj];
        if (a.v_prev[0]) {
            v0 = a.v_prev[0][bj];
            if constexpr (MODE != kPlain) v1 = a.v_prev[1][bj];
        }
        if constexpr (MODE == kAdam) {
            m1 = a.m1[bj];
            m2 = a.m2[bj];
        }
    }
    const Prev pv = previous_from(words, a.prev != nullptr, a.method, a.tol);
    if (pv.stop) return;
    bool keep = false;
    if constexpr (MODE != kPlain) keep = wave_max(g0) < wave_max(g1);
    float cs = keep ? cs_n : cs_t;
    fold[sl][jj] = cs;
#pragma unroll
    for (int half = kFoldLanes / 2; half >= 1; half /= 2) {
        __syncthreads();
        if (sl < half) {
            cs += fold[sl + half][jj];
            fold[sl][jj] = cs;
        }
    }
    float gap0 = 0.0f, gap1 = 0.0f, move = 0.0f;
    if (col) {
        const float vcur = MODE != kPlain && pv.d.keep_v ? v1 : v0;
        float vt;
        if (cs >= kColSumFloor && cs <= FLT_MAX) {
            vt = lgb + vcur - logf(cs);
        } else {
            // the reference's max-shifted column LSE (kernels.cu:629-671)
            const float* col = a.X + size_t(b) * a.M * a.N + j;
            const float* u = (keep ? a.un : a.ut) + size_t(b) * a.M;
            float mx = -FLT_MAX;
            for (int i = 0; i < a.M; ++i) mx = fmaxf(mx, fmaf(col[size_t(i) * a.N], a.kscale, u[i]));
            float sm = 0.0f;
            for (int i = 0; i < a.M; ++i) sm += safe_exp(fmaf(col[size_t(i) * a.N], a.kscale, u[i]) - mx);
            vt = lgb - (mx + logf(fmaxf(sm, kSumFloor)));
        }
        a.vt[bj] = vt;
        if constexpr (MODE != kPlain) {
            float vn;
            if constexpr (MODE == kMomentum) {
                vn = (1.0f - a.omega) * vcur + a.omega * vt;
            } else {
                const float g = vt - vcur;
                const float mm = a.beta1 * m1 + (1.0f - a.beta1) * g;
                const float vv = a.beta2 * m2 + (1.0f - a.beta2) * (g * g);
                a.m1[bj] = mm;
                a.m2[bj] = vv;
                vn = vcur + a.lr * (mm / a.c1) / (sqrtf(vv / a.c2) + a.eps);
            }
            a.vn[bj] = vn;
            gap0 = fabsf(vn - vt);
            gap1 = fabsf(vcur - vt);
            move = fabsf(vn - vcur);
        }
    }
    if constexpr (MODE != kPlain) block_flag_max<3>(a.slots, kGapV, gap0, kGapV + 1, gap1, kMoveV, move, red);
}

// ---------------------------------------------------------------------------
// End of the loop: iterations executed, and the potentials the last one kept.
// ---------------------------------------------------------------------------
// The sweeps count the iterations and flag a stop they find; a stop at the
// last iteration has no later sweep to find it (one wave).
static __global__ void finalize(const unsigned* last, int method, float tol, int32_t* converged) {
    const Decision d = decide_dev(last, method);
    if (threadIdx.x == 0 && tol > 0.0f && d.delta < tol) *converged = 1;
}

static __global__ void reset_counts(int32_t* used, int32_t* converged) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *used = 0;
        *converged = 0;
    }
}

struct ResolveArgs {
    int B, M, N, method;
    const int32_t* used;
    const unsigned* slots;
    const float* ut[2];  // by parity of the iteration
    const float* un[2];
    const float* vt[2];
    const float* vn[2];
    float* u;            // [B,M] out
    float* v;            // [B,N] out
};

static __global__ __launch_bounds__(kBlock) void resolve(ResolveArgs a) {
    const int T = *a.used;
    const size_t nu = size_t(a.B) * a.M, n = nu + size_t(a.B) * a.N;
    const unsigned* s = T > 0 ? a.slots + size_t(T - 1) * kIterWords : nullptr;
    const int p = (T - 1) & 1;
    const Decision d = s ? decide_dev(s, a.method) : Decision{false, false, 0.0f};
    const bool ku = d.keep_u, kv = d.keep_v;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        if (i < nu) a.u[i] = s ? (ku ? a.un[p] : a.ut[p])[i] : 0.0f;
        else a.v[i - nu] = s ? (kv ? a.vn[p] : a.vt[p])[i - nu] : 0.0f;
    }
}

// ---------------------------------------------------------------------------
// Anderson mixing (torch_cuda.cpp:395-446) on the state x = (u, v) of each
// batch element, with a ring of up to kMaxHistory (x, f = x_new - x) pairs.
// The Gram matrix F^T F of the ring is kept across iterations: a push adds
// the new residual's products with every pair in the ring (the others'
// products are unchanged), so an iteration reads the history once.
// ---------------------------------------------------------------------------
constexpr int kGramChunk = kBlock;  // state entries per push workgroup (one per thread)

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
    int order[kMaxHistory];  // physical slots, oldest first (the newest is order[h-1] = slot)
    float mixing_beta;
    float* dots;      // [B,nchunk,kMaxHistory] per-chunk products of the new residual with order[q]
    int nchunk;       // chunks of kGramChunk state entries
    float* gram;      // [B,kMaxHistory,kMaxHistory] by physical slot, kept across iterations
    float* alpha;     // [B,kMaxHistory]
    float* denom;     // [B]
    const unsigned* prev;
    unsigned* slots;  // this iteration's flag words
    float tol;
};

// Push (x, x_new - x) into the ring for one chunk of one element's state
// (grid nchunk x B), with the chunk's products of the new residual and every
// residual in the ring, and the residual's max into the delta word.
static __global__ __launch_bounds__(kBlock) void aa_push(AaArgs a) {
    __shared__ float red[3 * kWavesPerBlock];
    __shared__ float dred[kWavesPerBlock][kMaxHistory];
    if (previous(a.prev, kAnderson, a.tol).stop) return;
    const int ch = blockIdx.x, b = batch_of_block(), h = a.h;
    if (b >= a.B) return;
    const size_t nu = size_t(a.B) * a.M, nv = size_t(a.B) * a.N;
    const int i1 = min((ch + 1) * kGramChunk, a.M + a.N);
    float acc[kMaxHistory];
#pragma unroll
    for (int q = 0; q < kMaxHistory; ++q) acc[q] = 0.0f;
    float d = 0.0f;
    for (int i = ch * kGramChunk + threadIdx.x; i < i1; i += kBlock) {
        const bool isu = i < a.M;
        const size_t k = isu ? size_t(b) * a.M + i : size_t(b) * a.N + (i - a.M);
        const size_t st = isu ? nu : nv;
        const float x = isu ? a.xu[k] : a.xv[k];
        const float f = (isu ? a.nu[k] : a.nv[k]) - x;
        (isu ? a.hxu : a.hxv)[size_t(a.slot) * st + k] = x;
        (isu ? a.hfu : a.hfv)[size_t(a.slot) * st + k] = f;
        d = fmaxf(d, fabsf(f));
        const float* hf = isu ? a.hfu : a.hfv;
#pragma unroll
        for (int q = 0; q < kMaxHistory; ++q)
            if (q < h) acc[q] = fmaf(f, q == h - 1 ? f : hf[size_t(a.order[q]) * st + k], acc[q]);
    }
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
    for (int q = 0; q < kMaxHistory; ++q) {
        const float s = wave_sum(acc[q]);
        if (lane == 0) dred[wave][q] = s;
    }
    block_flag_max<1>(a.slots, kAaDelta, d, 0, 0.0f, 0, 0.0f, red);  // barrier for dred too
    if (threadIdx.x < h) {
        const int q = threadIdx.x;
        float s = dred[0][q];
#pragma unroll
        for (int w = 1; w < kWavesPerBlock; ++w) s += dred[w][q];
        a.dots[(size_t(b) * a.nchunk + ch) * kMaxHistory + q] = s;
    }
}

// One workgroup per element: fold the new products (chunks in order) into
// the kept Gram matrix, then (G + 1e-8 I) alpha = 1 over the ring (oldest
// first) by Gaussian elimination with partial pivoting (the updates of a
// column in parallel, one thread per entry; h <= kMaxHistory) and sum(alpha); a zero or non-finite pivot or sum marks the
// iteration's solve as failed.  With fewer than two pairs only the Gram
// matrix is updated.
static __global__ void aa_solve(AaArgs a) {
    __shared__ float A[kMaxHistory][kMaxHistory + 1];
    __shared__ float x[kMaxHistory];
    __shared__ float fresh[kMaxHistory];  // the new residual's products, by ring position
    if (previous(a.prev, kAnderson, a.tol).stop) return;
    const int b = blockIdx.x, h = a.h;
    float* G = a.gram + size_t(b) * kMaxHistory * kMaxHistory;
    if (threadIdx.x < h) {
        const int q = threadIdx.x;
        float s = 0.0f;
        for (int ch = 0; ch < a.nchunk; ++ch) s += a.dots[(size_t(b) * a.nchunk + ch) * kMaxHistory + q];
        fresh[q] = s;
        const int pq = a.order[q];
        G[a.slot * kMaxHistory + pq] = s;  // kept for later iterations
        G[pq * kMaxHistory + a.slot] = s;
    }
    __syncthreads();
    if (h < 2) return;
    // the newest pair is ring position h - 1; its products come from LDS, the
    // others' from the kept matrix (written by earlier launches)
    for (int e = threadIdx.x; e < h * h; e += blockDim.x) {
        const int p = e / h, q = e % h;
        const float g = p == h - 1 ? fresh[q]
                        : q == h - 1 ? fresh[p]
                                     : G[a.order[p] * kMaxHistory + a.order[q]];
        A[p][q] = g + (p == q ? 1.0e-8f : 0.0f);
    }
    if (threadIdx.x < h) x[threadIdx.x] = 1.0f;
    __shared__ float fr[kMaxHistory];
    __shared__ int piv_sh, fail_sh;
    // forward elimination: per column, the pivot by one thread, then the row
    // swap and the updates of the rows below, the entries spread over the threads
    for (int c = 0; c < h; ++c) {
        __syncthreads();
        if (threadIdx.x == 0) {
            int piv = c;
            for (int r = c + 1; r < h; ++r)
                if (fabsf(A[r][c]) > fabsf(A[piv][c])) piv = r;
            const float pv = A[piv][c];
            piv_sh = piv;
            fail_sh = (pv == 0.0f || !(fabsf(pv) <= FLT_MAX)) ? 1 : 0;
        }
        __syncthreads();
        if (fail_sh) break;
        const int piv = piv_sh;
        if (piv != c) {
            if (threadIdx.x < h) {
                const float t = A[c][threadIdx.x];
                A[c][threadIdx.x] = A[piv][threadIdx.x];
                A[piv][threadIdx.x] = t;
            } else if (threadIdx.x == kMaxHistory) {
                const float t = x[c];
                x[c] = x[piv];
                x[piv] = t;
            }
            __syncthreads();
        }
        if (threadIdx.x > c && threadIdx.x < h) fr[threadIdx.x] = A[threadIdx.x][c] / A[c][c];
        __syncthreads();
        const int rows = h - c - 1, cols = h - c;  // rows c+1 .. h-1, columns c .. h-1
        for (int e = threadIdx.x; e < rows * cols; e += blockDim.x) {
            const int tr = c + 1 + e / cols, tq = c + e % cols;
            A[tr][tq] -= fr[tr] * A[c][tq];
        }
        if (threadIdx.x > c && threadIdx.x < h) x[threadIdx.x] -= fr[threadIdx.x] * x[c];
    }
    __syncthreads();
    const bool failed_elim = fail_sh != 0;
    // back substitution, one column at a time
    if (!failed_elim) {
        for (int c = h - 1; c >= 0; --c) {
            if (threadIdx.x == 0) x[c] = x[c] / A[c][c];
            __syncthreads();
            if (threadIdx.x < c) x[threadIdx.x] -= A[threadIdx.x][c] * x[c];
            __syncthreads();
        }
    }
    if (threadIdx.x != 0) return;
    bool failed = failed_elim;
    float sum = 0.0f;
    if (!failed) {
        for (int c = 0; c < h; ++c) sum += x[c];
        failed = !(fabsf(sum) <= FLT_MAX);
    }
    for (int c = 0; c < h; ++c) a.alpha[size_t(b) * kMaxHistory + c] = failed ? 0.0f : x[c];
    a.denom[b] = sum;
    if (failed) atomicMax(a.slots + flag_at(kAaFail, b % kStripes), 1u);
    else atomicMax(a.slots + flag_at(kAaMin, b % kStripes), kInfBits - __float_as_uint(fabsf(sum)));
}

// x = sum_c (alpha_c / sum) (X_c + beta F_c) when every element's solve
// succeeded with |sum| >= 1e-12, else x = x_new (torch_cuda.cpp:421-444).
// With fewer than two pairs, x = x_new.
static __global__ __launch_bounds__(kBlock) void aa_update(AaArgs a) {
    if (previous(a.prev, kAnderson, a.tol).stop) return;
    // the stripes hold kInfBits - bits(|sum|): their max is the minimum |sum|
    const float fail = flag(a.slots, kAaFail);
    const float code = flag(a.slots, kAaMin);
    const bool mix = a.h >= 2 && fail == 0.0f &&
                     __uint_as_float(kInfBits - __float_as_uint(code)) >= 1.0e-12f;
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
    int B, M, N, rows, return_log;
    int nchunks;          // column chunks per row (1 unless N > kMaxRowLen)
    int safe;             // safe_exp (the vanilla materialisation) rather than exp
    const float* u;
    const float* v;
    float* plan;          // or null
    float* cost_partial;  // [B, nstrips * nchunks] or null
};

// One strip x chunk tile (tile.cuh) per workgroup; a whole row when nchunks is 1.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void plan(PlanArgs a) {
    using R = Row<VEC, CH>;
    __shared__ float scratch[kWavesPerBlock];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const wide::Tile tl = wide::tile_of_block(a.nchunks, a.N);
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    float v[R::PL];
    R::load(a.v + size_t(b) * a.N + tl.c0, lane, tl.nc, v, 0.0f);
    float cacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (size_t(b) * a.M + i) * a.N + tl.c0;
        float x[R::PL];
        R::load(a.X + off, lane, tl.nc, x, 0.0f);
        const float ui = a.u[size_t(b) * a.M + i];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float lp = x[e] * a.kscale + ui + v[e];
            const float p = a.return_log ? lp : (a.safe ? safe_exp(lp) : expf(lp));
            if (a.cost_partial && R::valid(lane, e, tl.nc)) cacc = fmaf(p, a.csign * x[e], cacc);
            x[e] = p;
        }
        if (a.plan) R::store(a.plan + off, lane, tl.nc, x);
    }
    if (a.cost_partial) {
        const float s = block_reduce<kWavesPerBlock>(wave_sum(cacc), scratch, OpSum{});
        if (threadIdx.x == 0) a.cost_partial[size_t(b) * gridDim.x + blockIdx.x] = s;
    }
}

}  // namespace mth
}  // namespace dot_amd
