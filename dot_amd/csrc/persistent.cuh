// Persistent streaming kernels: one cooperative launch for all iterations
// when a batch element's rows do not fit the registers of its workgroups.
//
// Each batch element gets W workgroups (one per CU, 8 waves), each owning a
// strip of rows that it streams from HBM / the Infinity Cache once per
// iteration, exactly like a streaming sweep, but without a kernel boundary
// between iterations.  The per-column sums go through a reduce-scatter and an
// all-gather of tagged words (see resident.cuh for the tag protocol):
//   1. the workgroup's column sums (fixed-order fold of its waves) are
//      published as one tagged row;
//   2. workgroup w owns the column slice [w N / W, (w+1) N / W): it reads the
//      W rows for its slice (every value in flight at once), adds them in
//      workgroup order and publishes the slice's results (v or mu);
//   3. every workgroup reads the N results of its element.
// Two memory round trips per iteration and 2 N + N / W tagged reads per
// workgroup, whatever W is.  Slots alternate by iteration parity; a workgroup
// cannot reach iteration t+2 before every owner has consumed iteration t.
#pragma once

#include <cfloat>
#include <cstdint>

#include "resident.cuh"

namespace dot_amd {
namespace pst {

using res::kThreads;
using res::kWaves;
using res::publish;
using res::tag_pack;

constexpr int kMaxGroups = 64;                                   // workgroups per batch element
constexpr int kMaxCols = kMaxRowLen;                             // 4096
constexpr int kLoadsPerThread = (kMaxCols + kMaxGroups + kThreads - 1) / kThreads;  // 9

// The lane index behind an empty asm: addresses and masks computed from it
// are recomputed where they are used instead of being hoisted out of the
// iteration loop (64-float rows would otherwise pin dozens of registers).
__device__ __forceinline__ int opaque_lane() {
    int lane = threadIdx.x % kWave;
    asm volatile("" : "+v"(lane));
    return lane;
}

__device__ __forceinline__ int slice_begin(int w, int W, int N) {
    return static_cast<int>(static_cast<long long>(w) * N / W);
}

// Polls `n` tagged words at base[idx(r)] (r < n <= kLoadsPerThread, all in flight)
// until each carries tag t; returns false after a timeout (values then NaN).
template <class Idx>
__device__ __forceinline__ bool poll_many(const unsigned long long* base, int n, Idx idx, unsigned t,
                                          int spin_limit, int* status, bool& dead,
                                          float (&out)[kLoadsPerThread]) {
    res::forced_timeout(spin_limit, status, dead);
    if (dead) {
#pragma unroll
        for (int r = 0; r < kLoadsPerThread; ++r) out[r] = __builtin_nanf("");
        return false;
    }
    for (int spins = 0;; ++spins) {
        bool ready = true;
#pragma unroll
        for (int r = 0; r < kLoadsPerThread; ++r) {
            if (r < n) {
                const unsigned long long x = __hip_atomic_load(
                    const_cast<unsigned long long*>(base + idx(r)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ready = ready && static_cast<unsigned>(x >> 32) == t;
                out[r] = __uint_as_float(static_cast<unsigned>(x));
            }
        }
        if (ready) return true;
        if (((spins & 255) == 255 &&
             __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) ||
            spins >= spin_limit) {
            if (spins >= spin_limit) atomicOr(status, 1);
            dead = true;
#pragma unroll
            for (int r = 0; r < kLoadsPerThread; ++r) out[r] = __builtin_nanf("");
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Per-column vectors (v, mu) as the row loops use them: rows of up to 32
// floats per lane keep the vector in registers; longer rows (N > 2048) read
// it from LDS one chunk at a time, which leaves the registers to the row and
// the column accumulator.
template <int VEC, int CH>
struct ColVec {
    static constexpr bool kLds = VEC * CH > 32;
    float reg[kLds ? 1 : VEC * CH];
    const float* lds;

    __device__ __forceinline__ void bind(const float* v, int lane, int N) {
        lds = v;
        if constexpr (!kLds) Row<VEC, CH>::load(v, lane, N, reg, 0.0f);
    }
    // columns k*64*VEC + lane*VEC + [0, VEC) of the vector (0 past N)
    __device__ __forceinline__ void chunk(int lane, int k, int N, float (&out)[VEC]) const {
        if constexpr (kLds) {
            const int c = Row<VEC, CH>::col(lane, k);
            if constexpr (VEC == 4) {  // N % 4 == 0: a chunk is all in or all out
                float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (c < N) t = *reinterpret_cast<const float4*>(lds + c);
                out[0] = t.x;
                out[1] = t.y;
                out[2] = t.z;
                out[3] = t.w;
            } else {
                out[0] = c < N ? lds[c] : 0.0f;
            }
        } else {
#pragma unroll
            for (int q = 0; q < VEC; ++q) out[q] = reg[k * VEC + q];
        }
    }
};

// LDS rows of the step-1 fold: all 8 waves' rows at once when a row is at most
// 32 floats per lane (publish_row_flat), else a halving tree through 4 rows.
template <int VEC, int CH>
constexpr int kFoldRows = VEC * CH <= 32 ? kWaves : kWaves / 2;

// Step 1 with every wave's row in LDS: one barrier, then thread t adds
// columns t, t + 512, ... over the 8 waves in order and publishes them, so
// the stores are spread over all 512 threads.  Contains barriers; `rows`
// holds 8 N floats.
template <int VEC, int CH>
__device__ __forceinline__ void publish_row_flat(const float (&acc)[VEC * CH], float* rows, int N,
                                                 unsigned long long* slot_row, unsigned t, bool local) {
    using R = Row<VEC, CH>;
    const int wave = threadIdx.x / kWave;
    __syncthreads();  // earlier readers of `rows` are done
    R::store(rows + wave * N, opaque_lane(), N, acc);
    __syncthreads();
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    for (int j = tid; j < N; j += kThreads) {
        float s = rows[j];
#pragma unroll
        for (int v = 1; v < kWaves; ++v) s += rows[v * N + j];
        publish(slot_row + j, s, t, local);
    }
}

// Step 1 through 4 LDS rows (rows of 64 floats per lane): waves 4..7 store,
// waves 0..3 add them to their own rows and store the pairs, then thread t
// adds columns t, t + 512, ... over the 4 pair rows in order and publishes
// them.  Contains barriers; `rows` holds 4 N floats.
template <int VEC, int CH>
__device__ __forceinline__ void publish_row_pairs(float (&acc)[VEC * CH], float* rows, int N,
                                                  unsigned long long* slot_row, unsigned t, bool local) {
    using R = Row<VEC, CH>;
    const int wave = threadIdx.x / kWave;
    constexpr int H = kWaves / 2;
    __syncthreads();  // earlier readers of `rows` are done
    if (wave >= H) R::store(rows + (wave - H) * N, opaque_lane(), N, acc);
    __syncthreads();
    if (wave < H) {
        const int ln = opaque_lane();
        float o[R::PL];
        R::load(rows + wave * N, ln, N, o, 0.0f);
#pragma unroll
        for (int e = 0; e < R::PL; ++e) acc[e] += o[e];
        R::store(rows + wave * N, ln, N, acc);
    }
    __syncthreads();
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    for (int j = tid; j < N; j += kThreads) {
        float s = rows[j];
#pragma unroll
        for (int v = 1; v < H; ++v) s += rows[v * N + j];
        publish(slot_row + j, s, t, local);
    }
}

// Step 1: fold the waves' per-lane column sums in a fixed order and publish
// the workgroup's row with tag t at slot_row (every thread publishes; `local`
// as for res::publish).
template <int VEC, int CH>
__device__ __forceinline__ void publish_row(float (&acc)[VEC * CH], float* tree, int N,
                                            unsigned long long* slot_row, unsigned t, bool local) {
    if constexpr (kFoldRows<VEC, CH> == kWaves)
        publish_row_flat<VEC, CH>(acc, tree, N, slot_row, t, local);
    else
        publish_row_pairs<VEC, CH>(acc, tree, N, slot_row, t, local);
}

// Step 2: the owner's sums over the element's W rows for its slice [c0, c1),
// in workgroup order.  `red` holds W * (c1 - c0) floats.  f(j, total) is called
// once per owned column by one thread.  Contains barriers.
template <class F>
__device__ __forceinline__ void reduce_slice(const unsigned long long* rows, int N, int W, int c0, int c1,
                                             unsigned t, float* red, int spin_limit, int* status,
                                             bool& dead, F&& f) {
    // An opaque copy of the thread index keeps the compiler from hoisting these
    // address computations out of the caller's iteration loop, where they
    // would hold registers through the whole row phase.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int S = c1 - c0;
    const int n = W * S;
    const int mine = n > tid ? (n - 1 - tid) / kThreads + 1 : 0;
    float got[kLoadsPerThread];
    poll_many(rows, mine,
              [&](int r) {
                  const int q = tid + r * kThreads;  // q = g * S + jj
                  return unsigned(q / S) * unsigned(N) + unsigned(c0 + q % S);
              },
              t, spin_limit, status, dead, got);
#pragma unroll
    for (int r = 0; r < kLoadsPerThread; ++r)
        if (r < mine) red[tid + r * kThreads] = got[r];
    __syncthreads();
    for (int jj = threadIdx.x; jj < S; jj += kThreads) {
        float s = 0.0f;
        for (int g = 0; g < W; ++g) s += red[g * S + jj];
        f(c0 + jj, dead ? __builtin_nanf("") : s);
    }
}

// Step 3: read the element's N published results into `out` (LDS).  The
// caller synchronises before reading `out`.
__device__ __forceinline__ void gather(const unsigned long long* res_row, int N, unsigned t, float* out,
                                       int spin_limit, int* status, bool& dead) {
    int tid = threadIdx.x;  // opaque, as in reduce_slice
    asm volatile("" : "+v"(tid));
    const int mine = N > tid ? (N - 1 - tid) / kThreads + 1 : 0;
    float got[kLoadsPerThread];
    poll_many(res_row, mine, [&](int r) { return unsigned(tid + r * kThreads); }, t, spin_limit, status, dead,
              got);
#pragma unroll
    for (int r = 0; r < kLoadsPerThread; ++r)
        if (r < mine) out[tid + r * kThreads] = got[r];
}

// gather() of a row that carries W more words after its N results (one per
// slice owner), which are not stored: returns this thread's largest
// |new - old| over the N results (old: what `out` held before) and its
// largest extra word.
__device__ __forceinline__ void gather_track(const unsigned long long* res_row, int N, int W, unsigned t,
                                             float* out, int spin_limit, int* status, bool& dead, float& dmax,
                                             float& xmax) {
    int tid = threadIdx.x;  // opaque, as in reduce_slice
    asm volatile("" : "+v"(tid));
    const int n = N + W;
    const int mine = n > tid ? (n - 1 - tid) / kThreads + 1 : 0;
    float got[kLoadsPerThread];
    poll_many(res_row, mine, [&](int r) { return unsigned(tid + r * kThreads); }, t, spin_limit, status, dead,
              got);
#pragma unroll
    for (int r = 0; r < kLoadsPerThread; ++r) {
        const int j = tid + r * kThreads;
        if (r < mine && j < N) {
            dmax = fmaxf(dmax, fabsf(got[r] - out[j]));
            out[j] = got[r];
        } else if (r < mine) {
            xmax = fmaxf(xmax, got[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
struct FwdArgs {
    const float* X;       // scores [B,M,N]
    float kscale;         // K = X * kscale (the plan's; every iteration's unless scheduled)
    const float* kscale_t;  // [max_iter] K scale of each iteration (tau schedule), SCHED kernels
    int scores_kind;      // +1 log_alpha, -1 cost
    const float* log_a;   // [B,M] or null
    const float* log_b;   // [B,N] or null
    float log_a_default, log_b_default;
    float tol;
    int max_iter;
    int return_log;
    float* plan;          // [B,M,N] or null
    float* cost_partial;  // [G] by logical workgroup, or null
    float* u_out;         // [B,M] or null
    float* v_out;         // [B,N] or null
    float* u_hist;        // [T,B,M] or null
    float* v_hist;        // [T,B,N] or null
    int32_t* iters_used;
    int32_t* converged;
    unsigned long long* part;   // [2, G, N] tagged workgroup column sums
    unsigned long long* res;    // [2, B, N] tagged new v
    unsigned long long* uslot;  // [2, B, M] tagged u (read by the exact column LSE)
    unsigned long long* dxchg;  // [kDeltaSlots, G] tagged per-workgroup deltas
    int* status;
    int B, M, N, W, R, spin_limit;
    int local_ok;         // XCD-local exchange stores allowed (local_exchange_allowed)
    float* ebuf;                // [B,M,N] scaled kernel (scaling domain), or null
};

// Dual Sinkhorn forward (torch_cuda.cpp:147-264), streaming each workgroup's
// strip once per iteration.  Row update in base 2 as in res::forward (one
// wave per row), the shared-exponential column sums, reduce-scatter to the
// slice owners, who form v_j = log b_j + v_j - log colsum_j (or the exact
// max-shifted LSE of column j over all M rows when colsum underflows,
// kernels.cu:629-671), all-gather of v.  The batch-global stop test of
// iteration t-1 is read during iteration t, as in res::forward.
//
// Scaling domain (ebuf set, one K scale for every iteration): the workgroup
// first writes E_ij = 2^(x_ij kscale log2(e) - mx_i) for its rows (mx_i: the
// row's maximum) and then streams E instead of the scores: with V_j =
// 2^(v_j log2(e) - mv) (mv: the maximum over columns), s_i = sum_j E_ij V_j,
// u_i = log a_i - ln2 (mx_i + mv + log2 s_i), and the column sums are
// V_j sum_i E_ij a_i / s_i -- the sums of exp(K + u + v) the log-domain update
// forms, at two FMAs per element instead of an exponential and a maximum.  The
// largest term of a row is at least 2^-(max_j v - min_j v) log2(e), so while
// that range is within kScalingRange every kept term is exact to float
// precision; past it the workgroup streams the scores in the log domain for
// the remaining iterations.  The exact column LSE and the plan read the scores.
// Rows of 64 floats per lane (N > 2048), which are processed one at a time,
// gain (C5: 42.5 -> 40.6 us per iteration).
constexpr float kScalingRange = 64.0f;  // log2 units

template <int VEC, int CH, bool SCHED = false>
__global__ __launch_bounds__(kThreads) void forward(FwdArgs a) {
    using R = Row<VEC, CH>;
    constexpr int PL = R::PL;
    // LDS: fold (kFoldRows) N | v N | v log2(e) N | log b N | red N + W (padded to 4) | u 2R | log a R | scratch 32
    extern __shared__ float lds[];
    float* tree = lds;
    float* lds_v = tree + kFoldRows<VEC, CH> * a.N;
    float* lds_v2 = lds_v + a.N;
    float* lds_lb = lds_v2 + a.N;
    float* red = lds_lb + a.N;
    float* lds_u = red + ((a.N + a.W + 3) & ~3);
    float* lds_la = lds_u + 2 * a.R;
    float* lds_mx = lds_la + a.R;  // scaling domain: row maxima of x kscale log2(e)
    float* scratch = lds_mx + a.R;  // [0] global delta, [1..kWaves] wave deltas, [16..] reductions
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int G = gridDim.x;
    const int gid = res::logical_group(a.W);
    const int b = gid / a.W;
    const int w = gid % a.W;
    const int row0 = w * a.R;
    const int rend = min(row0 + a.R, a.M);
    const int c0 = slice_begin(w, a.W, a.N), c1 = slice_begin(w + 1, a.W, a.N);
    const size_t bM = size_t(b) * a.M;
    const size_t bN = size_t(b) * a.N;
    const bool check = a.tol > 0.0f;
    float kscale2 = a.kscale * kLog2E;
    // scheduled runs: this iteration's scale, and the next one's already in flight
    float ks_it = a.kscale;
    float ks_next = (SCHED && a.max_iter > 0) ? a.kscale_t[0] : a.kscale;
    res::announce_xcc(a.part, a.N, b, a.W, w);

    for (int l = threadIdx.x; l < a.R; l += kThreads) {
        const int i = row0 + l;
        lds_la[l] = (i < rend && a.log_a) ? a.log_a[bM + i] : a.log_a_default;
        lds_u[l] = 0.0f;
        lds_u[a.R + l] = 0.0f;
    }
    // (rows of 64 floats per lane only: the pipelined rows of up to 32 floats
    // hide their arithmetic under the stream already -- C4 lost 1 us per
    // iteration to the scaling domain's per-iteration range reduction)
    bool scal = !SCHED && PL > 32 && a.ebuf != nullptr;
    float mv = 0.0f;  // scaling domain: lds_v2 holds V = 2^(v log2(e) - mv)
    for (int j = threadIdx.x; j < a.N; j += kThreads) {
        lds_lb[j] = a.log_b ? a.log_b[bN + j] : a.log_b_default;
        lds_v[j] = 0.0f;
        lds_v2[j] = scal ? 1.0f : 0.0f;
    }
    if (scal) {
        // E rows of this workgroup, each written and later read by the same wave
        for (int l = wave; l < rend - row0; l += kWaves) {
            const int ln = opaque_lane();
            float x[PL];
            R::load(a.X + (bM + row0 + l) * a.N, ln, a.N, x, 0.0f);
            float ml = -FLT_MAX;
#pragma unroll
            for (int e = 0; e < PL; ++e) {
                x[e] = R::valid(ln, e, a.N) ? x[e] * kscale2 : -INFINITY;
                ml = fmaxf(ml, x[e]);
            }
            const float m = wave_max(ml);
#pragma unroll
            for (int e = 0; e < PL; ++e) x[e] = __builtin_amdgcn_exp2f(x[e] - m);  // 0 for -inf
            R::store(a.ebuf + (bM + row0 + l) * a.N, ln, a.N, x);
            if (ln == 0) lds_mx[l] = m;
        }
    }
    __syncthreads();
    bool dead = false;
    const bool local =
        res::element_on_one_xcd(a.part, a.N, b, a.W, w, a.spin_limit, a.status, dead, scratch) && a.local_ok;
    int used = a.max_iter;
    int conv = 0;

    for (int t = 1; t <= a.max_iter; ++t) {
        const int cur = t & 1, prev = cur ^ 1;
        const bool test = check && t >= 2;
        if constexpr (SCHED) {
            ks_it = ks_next;
            kscale2 = ks_it * kLog2E;
            if (t < a.max_iter) ks_next = a.kscale_t[t];
        }
        unsigned long long* ds = a.dxchg + size_t((t - 1) % res::kDeltaSlots) * G;
        unsigned long long dpre[res::kDeltaPrefetch];
        if (test && wave == 0) {
#pragma unroll
            for (int q = 0; q < res::kDeltaPrefetch; ++q) {
                const int g = lane + q * kWave;
                dpre[q] = g < G ? __hip_atomic_load(ds + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : tag_pack(0.0f, unsigned(t - 1));
            }
        }
        ColVec<VEC, CH> v2;
        v2.bind(lds_v2, lane, a.N);
        float acc[PL];
#pragma unroll
        for (int e = 0; e < PL; ++e) acc[e] = 0.0f;
        float dmax = 0.0f;
        // rows of up to 32 floats per lane: each row's load is issued one row ahead
        auto load_row = [&](int l, RowBuf<R>& buf) {
            R::load_clamped(a.X + (bM + row0 + l) * a.N, opaque_lane(), a.N, buf.v, 0.0f);
        };
        auto row = [&](int l, RowBuf<R>& buf) {
            const int i = row0 + l;
            const int ln = opaque_lane();
            float(&y)[PL] = buf.v;
            float ml = -FLT_MAX;
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float vv[VEC];
                v2.chunk(ln, k, a.N, vv);
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    const int e = k * VEC + q;
                    y[e] = R::valid(ln, e, a.N) ? fmaf(y[e], kscale2, vv[q]) : -INFINITY;
                    ml = fmaxf(ml, y[e]);
                }
            }
            const float m = wave_max(ml);
            float sl = 0.0f;
#pragma unroll
            for (int e = 0; e < PL; ++e) {
                y[e] = __builtin_amdgcn_exp2f(y[e] - m);
                sl += y[e];
            }
            const float s = fmaxf(wave_sum(sl), sk::kSumFloor);
            const float lga = lds_la[l];
            const float lg2 = __builtin_amdgcn_logf(s);
            const float u = lga - kLn2 * (m + lg2);
            const float wgt = __builtin_amdgcn_exp2f(fmaf(lga, kLog2E, -lg2));
#pragma unroll
            for (int e = 0; e < PL; ++e) acc[e] = fmaf(y[e], wgt, acc[e]);
#pragma unroll
            for (int e = 0; e < PL; ++e) asm volatile("" : "+v"(acc[e]));  // keep the update here
            dmax = fmaxf(dmax, fabsf(u - lds_u[prev * a.R + l]));
            if (lane == 0) {
                lds_u[cur * a.R + l] = u;
                publish(a.uslot + size_t(cur) * a.B * a.M + bM + i, u, unsigned(t), local);
                if (a.u_hist) a.u_hist[(size_t(t - 1) * a.B + b) * a.M + i] = u;
            }
        };
        // scaling domain: the E row, s = sum E V, and the column partials sum E a / s
        auto load_row_e = [&](int l, RowBuf<R>& buf) {
            R::load_clamped(a.ebuf + (bM + row0 + l) * a.N, opaque_lane(), a.N, buf.v, 0.0f);
        };
        auto row_e = [&](int l, RowBuf<R>& buf) {
            const int i = row0 + l;
            const int ln = opaque_lane();
            float(&ev)[PL] = buf.v;
            float sl = 0.0f;
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float vv[VEC];
                v2.chunk(ln, k, a.N, vv);  // V, 0 past N
#pragma unroll
                for (int q = 0; q < VEC; ++q) sl = fmaf(ev[k * VEC + q], vv[q], sl);
            }
            const float s_sum = wave_sum(sl);
            const float s = s_sum > 0.0f ? s_sum : sk::kSumFloor;  // 0: a row with no finite K
            const float lga = lds_la[l];
            const float lg2 = __builtin_amdgcn_logf(s);
            const float u = lga - kLn2 * ((lds_mx[l] + mv) + lg2);
            const float wgt = __builtin_amdgcn_exp2f(fmaf(lga, kLog2E, -lg2));
#pragma unroll
            for (int e = 0; e < PL; ++e) acc[e] = fmaf(ev[e], wgt, acc[e]);
#pragma unroll
            for (int e = 0; e < PL; ++e) asm volatile("" : "+v"(acc[e]));  // keep the update here
            dmax = fmaxf(dmax, fabsf(u - lds_u[prev * a.R + l]));
            if (lane == 0) {
                lds_u[cur * a.R + l] = u;
                publish(a.uslot + size_t(cur) * a.B * a.M + bM + i, u, unsigned(t), local);
                if (a.u_hist) a.u_hist[(size_t(t - 1) * a.B + b) * a.M + i] = u;
            }
        };
        if (scal) {
            if constexpr (PL <= 32) {
                pipelined_rows<RowBuf<R>>(wave, rend - row0, kWaves, load_row_e, row_e);
            } else {
                for (int l = wave; l < rend - row0; l += kWaves) {
                    RowBuf<R> buf;
                    load_row_e(l, buf);
                    row_e(l, buf);
                }
            }
            // times V: the partials of exp(K + u + v) that the log-domain rows form
            const int ln = opaque_lane();
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float vv[VEC];
                v2.chunk(ln, k, a.N, vv);
#pragma unroll
                for (int q = 0; q < VEC; ++q) acc[k * VEC + q] *= vv[q];
            }
        } else if constexpr (PL <= 32) {
            pipelined_rows<RowBuf<R>>(wave, rend - row0, kWaves, load_row, row);
        } else {  // 64-float rows: a second buffer would spill
            for (int l = wave; l < rend - row0; l += kWaves) {
                RowBuf<R> buf;
                load_row(l, buf);
                row(l, buf);
            }
        }
        if (lane == 0) scratch[1 + wave] = dmax;
        publish_row<VEC, CH>(acc, tree, a.N, a.part + (size_t(cur) * G + gid) * a.N, unsigned(t), local);
        if (check && threadIdx.x == 0) {
            float d = scratch[1];
#pragma unroll
            for (int q = 1; q < kWaves; ++q) d = fmaxf(d, scratch[1 + q]);
            publish(a.dxchg + size_t(t % res::kDeltaSlots) * G + gid, d, unsigned(t));
        }
        unsigned long long* res_row = a.res + (size_t(cur) * a.B + b) * a.N;
        const unsigned long long* urow = a.uslot + size_t(cur) * a.B * a.M + bM;
        reduce_slice(a.part + size_t(cur) * G * a.N + size_t(b) * a.W * a.N, a.N, a.W, c0, c1, unsigned(t),
                     red, a.spin_limit, a.status, dead, [&](int j, float cs) {
                         float vn;
                         if (cs >= sk::kColSumFloor && cs <= FLT_MAX) {
                             vn = lds_lb[j] + lds_v[j] - logf(cs);
                         } else {
                             // exact max-shifted LSE over the column (kernels.cu:629-671)
                             const float* col = a.X + bM * a.N + j;
                             float mx = -FLT_MAX;
                             for (int i = 0; i < a.M; ++i) {
                                 const float ui = res::collect(const_cast<unsigned long long*>(urow + i), unsigned(t),
                                                               a.spin_limit, a.status, dead);
                                 mx = fmaxf(mx, col[size_t(i) * a.N] * ks_it + ui);
                             }
                             float sm = 0.0f;
                             for (int i = 0; i < a.M; ++i) {
                                 const float ui = __uint_as_float(static_cast<unsigned>(__hip_atomic_load(
                                     const_cast<unsigned long long*>(urow + i), __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT)));
                                 sm += safe_exp(col[size_t(i) * a.N] * ks_it + ui - mx);
                             }
                             vn = lds_lb[j] - (mx + logf(fmaxf(sm, sk::kSumFloor)));
                         }
                         publish(res_row + j, vn, unsigned(t), local);
                         if (a.v_hist) a.v_hist[(size_t(t - 1) * a.B + b) * a.N + j] = vn;
                     });
        __syncthreads();  // the owners have read lds_v (v_{t-1}); it now receives v_t
        gather(res_row, a.N, unsigned(t), lds_v, a.spin_limit, a.status, dead);
        if (scal) {  // stays in the scaling domain while max v - min v (log2) is within range
            float hi = -FLT_MAX, nlo = -FLT_MAX;
            for (int j = threadIdx.x; j < a.N; j += kThreads) {  // own writes
                const float q = lds_v[j] * kLog2E;
                hi = fmaxf(hi, q);
                nlo = fmaxf(nlo, -q);
            }
            hi = block_reduce<kWaves>(wave_max(hi), scratch + 16, OpMax{});
            nlo = block_reduce<kWaves>(wave_max(nlo), scratch + 16, OpMax{});
            scal = hi + nlo <= kScalingRange;  // false for NaN
            mv = hi;
        }
        for (int j = threadIdx.x; j < a.N; j += kThreads)  // own writes
            lds_v2[j] = scal ? __builtin_amdgcn_exp2f(fmaf(lds_v[j], kLog2E, -mv)) : lds_v[j] * kLog2E;
        if (test && wave == 0) {
            float gmax = 0.0f;
#pragma unroll
            for (int q = 0; q < res::kDeltaPrefetch; ++q) {
                const int g = lane + q * kWave;
                if (g < G) {
                    float d = __uint_as_float(static_cast<unsigned>(dpre[q]));
                    if (static_cast<unsigned>(dpre[q] >> 32) != unsigned(t - 1))
                        d = res::collect(ds + g, unsigned(t - 1), a.spin_limit, a.status, dead);
                    gmax = res::OpMaxNan{}(gmax, d);
                }
            }
            for (int g = lane + res::kDeltaPrefetch * kWave; g < G; g += kWave)
                gmax = res::OpMaxNan{}(gmax, res::collect(ds + g, unsigned(t - 1), a.spin_limit, a.status, dead));
            gmax = wave_reduce(gmax, res::OpMaxNan{});
            if (lane == 0) scratch[0] = gmax;
        }
        __syncthreads();
        if (test && scratch[0] < a.tol) {  // the stop test of iteration t-1 fired: back to v_{t-1}
            used = t - 1;
            conv = 1;
            __syncthreads();
            gather(a.res + (size_t(prev) * a.B + b) * a.N, a.N, unsigned(t - 1), lds_v, a.spin_limit,
                   a.status, dead);
            __syncthreads();
            break;
        }
    }
    if (check && conv == 0 && a.max_iter >= 1) {
        // the last iteration's deltas decide `converged`
        const unsigned T = unsigned(a.max_iter);
        unsigned long long* ds = a.dxchg + size_t(a.max_iter % res::kDeltaSlots) * G;
        if (wave == 0) {
            float m = 0.0f;
            for (int g = lane; g < G; g += kWave)
                m = res::OpMaxNan{}(m, res::collect(ds + g, T, a.spin_limit, a.status, dead));
            m = wave_reduce(m, res::OpMaxNan{});
            if (lane == 0) scratch[0] = m;
        }
        __syncthreads();
        conv = scratch[0] < a.tol ? 1 : 0;
    }

    // P = safe_exp(K + u + v) (kernels.cu:755-775) and this workgroup's share of sum(P C).
    const int par = used & 1;
    const bool failed = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    ColVec<VEC, CH> vf;
    vf.bind(lds_v, lane, a.N);
    if (a.v_out && w == 0)
        for (int j = threadIdx.x; j < a.N; j += kThreads) a.v_out[bN + j] = lds_v[j];
    const float csign = a.scores_kind < 0 ? 1.0f : -1.0f;  // C = -log_alpha
    float cacc = 0.0f;
    for (int l = wave; row0 + l < rend; l += kWaves) {
        const int i = row0 + l;
        const float ui = lds_u[par * a.R + l];
        if (a.u_out && lane == 0) a.u_out[bM + i] = ui;
        const int ln = opaque_lane();
        float x[PL];
        R::load(a.X + (bM + i) * a.N, ln, a.N, x, 0.0f);
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            float vv[VEC];
            vf.chunk(ln, k, a.N, vv);
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
                const int e = k * VEC + q;
                const float lp = (x[e] * a.kscale + ui) + vv[q];
                const float pe = a.return_log ? lp : safe_exp(lp);
                if (a.cost_partial && R::valid(ln, e, a.N)) cacc = fmaf(pe, csign * x[e], cacc);
                x[e] = failed ? __builtin_nanf("") : pe;
            }
        }
        if (a.plan) R::store(a.plan + (bM + i) * a.N, ln, a.N, x);
    }
    if (a.cost_partial) {
        const float cs = block_reduce<kWaves>(wave_sum(cacc), scratch + 16, OpSum{});
        if (threadIdx.x == 0) a.cost_partial[gid] = failed ? __builtin_nanf("") : cs;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *a.iters_used = failed ? -1 : used;  // -1: an exchange timed out, the outputs are NaN
        *a.converged = conv;
    }
}

// ---------------------------------------------------------------------------
// Implicit adjoint
// ---------------------------------------------------------------------------
struct ImpArgs {
    const float* X;
    int scores_kind;
    const float* gP;      // [B,M,N] or null
    const float* gC;      // [B] or null
    int gc_step;          // 1, or 0: gC holds one value for every batch element
    const float* P;       // [B,M,N]
    unsigned long long* part;  // [2, G, N] tagged workgroup column sums
    unsigned long long* res;   // [2, B, N + kMaxGroups] tagged mu, then each slice owner's stop-test scale
    unsigned long long* pro;   // [2, G, N] tagged prologue sums (P G, P)
    float* grad;
    float* tau_partial;   // [G] by logical workgroup
    int* status;
    float inv_tau;
    int B, M, N, W, R, iters, spin_limit;
    int local_ok;         // XCD-local exchange stores allowed (local_exchange_allowed)
    int32_t* sweeps;      // [B] sweeps executed per batch element, or null
    int early;            // nonzero: end each element's sweeps once converged (sk::AdjointStop)
};

template <int VEC, int CH>
__device__ __forceinline__ void upstream(const ImpArgs& a, size_t off, int lane, float gc, float csign,
                                         float (&x)[VEC * CH], float (&G)[VEC * CH]) {
    using R = Row<VEC, CH>;
    R::load(a.X + off, lane, a.N, x, 0.0f);
    if (a.gP) {
        R::load(a.gP + off, lane, a.N, G, 0.0f);
    } else {
#pragma unroll
        for (int e = 0; e < R::PL; ++e) G[e] = 0.0f;
    }
    if (a.gC) {
#pragma unroll
        for (int e = 0; e < R::PL; ++e) G[e] += gc * (csign * x[e]);
    }
}

// The implicit adjoint (kernels.cu:965-1098) streaming P once per sweep:
// prologue r, rs (rows) and c, cs (slice owners); per sweep lambda_i for the
// workgroup's rows, column sums of P lambda, reduce-scatter to the owners who
// form mu_k = (c_k - sum) / max(cs_k, 1e-12), all-gather of mu; final phase
// grad = P (G - lambda - mu) / tau (log-alpha kind: that - grad_cost P; cost
// kind: grad_cost P - that) and the workgroup's share of sum(grad * log_alpha).
// With `early`, an element's sweeps end once sk::AdjointStop finds them
// converged: the slice owners publish their slice's largest
// (|c_k| + |sum_i P lambda_i|) / cs_k after their mu, and every workgroup
// gathers those W words with mu, so all of them decide on the same values.
template <int VEC, int CH>
__global__ __launch_bounds__(kThreads) void implicit_adjoint(ImpArgs a) {
    using R = Row<VEC, CH>;
    constexpr int PL = R::PL;
    // LDS: fold (kFoldRows) N | mu N | red N + W | r R | 1/rs R | lambda R | c S | cs S | scratch 32
    extern __shared__ float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int G = gridDim.x;
    const int gid = res::logical_group(a.W);
    const int b = gid / a.W;
    const int w = gid % a.W;
    const int row0 = w * a.R;
    const int rend = min(row0 + a.R, a.M);
    const int c0 = slice_begin(w, a.W, a.N), c1 = slice_begin(w + 1, a.W, a.N);
    const int S = (a.N + a.W - 1) / a.W;
    float* tree = lds;
    float* lds_mu = tree + kFoldRows<VEC, CH> * a.N;
    float* red = lds_mu + a.N;
    float* lds_r = red + a.N + a.W;
    float* lds_irs = lds_r + a.R;
    float* lds_lam = lds_irs + a.R;
    float* lds_c = lds_lam + a.R;
    float* lds_cs = lds_c + S;
    float* scratch = lds_cs + S;
    const size_t bM = size_t(b) * a.M;
    const bool cost_kind = a.scores_kind < 0;
    const float gc = a.gC ? a.gC[b * a.gc_step] : 0.0f;
    const float csign = cost_kind ? 1.0f : -1.0f;  // C = csign * scores
    bool dead = false;
    res::announce_xcc(a.part, a.N, b, a.W, w);

    // Prologue: row sums of P G and P; column sums to the slice owners.
    float cg[PL], cp[PL];
#pragma unroll
    for (int e = 0; e < PL; ++e) cg[e] = cp[e] = 0.0f;
    for (int l = wave; row0 + l < rend; l += kWaves) {
        const size_t off = (bM + row0 + l) * a.N;
        const int ln = opaque_lane();
        float p[PL], x[PL], Gr[PL];
        R::load(a.P + off, ln, a.N, p, 0.0f);
        upstream<VEC, CH>(a, off, ln, gc, csign, x, Gr);
        float sg = 0.0f, sp = 0.0f;
#pragma unroll
        for (int e = 0; e < PL; ++e) {
            sg = fmaf(p[e], Gr[e], sg);
            sp += p[e];
            cg[e] = fmaf(p[e], Gr[e], cg[e]);
            cp[e] += p[e];
        }
        sg = wave_sum(sg);
        sp = wave_sum(sp);
        if (lane == 0) {
            lds_r[l] = sg;
            lds_irs[l] = 1.0f / fmaxf(sp, sk::kSumFloor);
            lds_lam[l] = 0.0f;
        }
    }
    const bool local =
        res::element_on_one_xcd(a.part, a.N, b, a.W, w, a.spin_limit, a.status, dead, scratch) && a.local_ok;
    publish_row<VEC, CH>(cg, tree, a.N, a.pro + size_t(gid) * a.N, 1u, local);
    publish_row<VEC, CH>(cp, tree, a.N, a.pro + (size_t(G) + gid) * a.N, 1u, local);
    reduce_slice(a.pro + size_t(b) * a.W * a.N, a.N, a.W, c0, c1, 1u, red, a.spin_limit, a.status, dead,
                 [&](int j, float tot) { lds_c[j - c0] = tot; });
    __syncthreads();
    reduce_slice(a.pro + (size_t(G) + size_t(b) * a.W) * a.N, a.N, a.W, c0, c1, 1u, red, a.spin_limit,
                 a.status, dead, [&](int j, float tot) { lds_cs[j - c0] = fmaxf(tot, sk::kSumFloor); });
    for (int j = threadIdx.x; j < a.N; j += kThreads) lds_mu[j] = 0.0f;
    __syncthreads();

    // Sweeps.
    sk::AdjointStop stop;
    int done_t = a.iters;
    for (int t = 1; t <= a.iters; ++t) {
        const int cur = t & 1;
        ColVec<VEC, CH> mu;
        mu.bind(lds_mu, lane, a.N);
        float acc[PL];
#pragma unroll
        for (int e = 0; e < PL; ++e) acc[e] = 0.0f;
        for (int l = wave; row0 + l < rend; l += kWaves) {
            const int ln = opaque_lane();
            float p[PL];
            R::load(a.P + (bM + row0 + l) * a.N, ln, a.N, p, 0.0f);
            float d = 0.0f;
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float mm[VEC];
                mu.chunk(ln, k, a.N, mm);
#pragma unroll
                for (int q = 0; q < VEC; ++q) d = fmaf(p[k * VEC + q], mm[q], d);
            }
            const float lam = (lds_r[l] - wave_sum(d)) * lds_irs[l];
#pragma unroll
            for (int e = 0; e < PL; ++e) acc[e] = fmaf(p[e], lam, acc[e]);
            if (lane == 0) lds_lam[l] = lam;
        }
        publish_row<VEC, CH>(acc, tree, a.N, a.part + (size_t(cur) * G + gid) * a.N, unsigned(t), local);
        unsigned long long* res_row = a.res + (size_t(cur) * a.B + b) * (size_t(a.N) + kMaxGroups);
        float sl = 0.0f;  // this thread's largest (|c_k| + |sum_i P lambda_i|) / cs_k of the slice
        reduce_slice(a.part + size_t(cur) * G * a.N + size_t(b) * a.W * a.N, a.N, a.W, c0, c1, unsigned(t),
                     red, a.spin_limit, a.status, dead, [&](int j, float tot) {
                         const float cj = lds_c[j - c0], csj = lds_cs[j - c0];
                         sl = fmaxf(sl, (fabsf(cj) + fabsf(tot)) / csj);
                         publish(res_row + j, (cj - tot) / csj, unsigned(t), local);
                     });
        if (a.early) {
            // stop-test values live at scratch + 16: block_reduce uses the first 8
            sl = block_reduce<kWaves>(wave_max(sl), scratch, OpMax{});
            if (threadIdx.x == 0) publish(res_row + a.N + w, sl, unsigned(t), local);
            float dmu = 0.0f, smu = 0.0f;
            gather_track(res_row, a.N, a.W, unsigned(t), lds_mu, a.spin_limit, a.status, dead, dmu, smu);
            dmu = wave_max(dmu);
            smu = wave_max(smu);
            // the last readers of these words are behind the barriers of the
            // next sweep's publish_row
            if (lane == 0) {
                scratch[16 + wave] = dmu;
                scratch[16 + kWaves + wave] = smu;
            }
        } else {
            gather(res_row, a.N, unsigned(t), lds_mu, a.spin_limit, a.status, dead);
        }
        __syncthreads();
        if (a.early && t < a.iters) {
            float d = scratch[16], sm = scratch[16 + kWaves];
#pragma unroll
            for (int q = 1; q < kWaves; ++q) {
                d = fmaxf(d, scratch[16 + q]);
                sm = fmaxf(sm, scratch[16 + kWaves + q]);
            }
            if (stop.done(t, d, sm)) {
                done_t = t;
                break;
            }
        }
    }
    if (a.sweeps && w == 0 && threadIdx.x == 0) a.sweeps[b] = done_t;

    // Final phase: stream P and G again and write this workgroup's gradient rows.
    const bool failed = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    ColVec<VEC, CH> mu;
    mu.bind(lds_mu, lane, a.N);
    float tacc = 0.0f;
    for (int l = wave; row0 + l < rend; l += kWaves) {
        const size_t off = (bM + row0 + l) * a.N;
        const float lam = lds_lam[l];
        const int ln = opaque_lane();
        float p[PL], x[PL], Gr[PL];
        R::load(a.P + off, ln, a.N, p, 0.0f);
        upstream<VEC, CH>(a, off, ln, gc, csign, x, Gr);
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            float mm[VEC];
            mu.chunk(ln, k, a.N, mm);
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
                const int e = k * VEC + q;
                const float gl = (p[e] * ((Gr[e] - lam) - mm[q])) * a.inv_tau;
                const float la = cost_kind ? -x[e] : x[e];
                if (R::valid(ln, e, a.N)) tacc = fmaf(gl, la, tacc);
                p[e] = failed ? __builtin_nanf("") : (cost_kind ? gc * p[e] - gl : gl - gc * p[e]);
            }
        }
        R::store_stream(a.grad + off, ln, a.N, p);
    }
    const float tsum = block_reduce<kWaves>(wave_sum(tacc), scratch, OpSum{});
    if (threadIdx.x == 0) a.tau_partial[gid] = failed ? __builtin_nanf("") : tsum;
}

// ---------------------------------------------------------------------------
// Unrolled backward
// ---------------------------------------------------------------------------
struct UnrArgs {
    const float* X;        // scores [B,M,N]
    int scores_kind;
    float kscale;          // K = X * kscale
    const float* gP;       // [B,M,N] or null
    const float* gC;       // [B] or null
    int gc_step;           // 1, or 0: gC holds one value for every batch element
    const float* P;        // [B,M,N]
    const float* u_hist;   // [T,B,M]
    const float* v_hist;   // [T,B,N]
    float* gamma;          // [B,M,N] Gamma between steps
    unsigned long long* part;  // [2, G, N] tagged workgroup column sums
    unsigned long long* res;   // [2, B, N] tagged column sums of the element
    float* grad;
    float* tau_partial;    // [G] by logical workgroup: sum(Gamma * log_alpha)
    int* status;
    float inv_tau;
    int B, M, N, W, R, T, spin_limit;
    int local_ok;          // XCD-local exchange stores allowed (local_exchange_allowed)
};

// The unrolled backward (kernels.cu:1622-1680) streaming Gamma and the scores
// once per reverse step: Gamma = G P; then for t = T-1 .. 0
//   Gamma_Y = Gamma - safe_exp(K + u_t + v_t) colsum(Gamma)
//   Gamma   = Gamma_Y - safe_exp(K + u_t + v_{t-1}) rowsum(Gamma_Y)
// with colsum(Gamma) from the reduce-scatter / all-gather of the previous
// step; the last step writes grad = Gamma / tau (log-alpha kind: that -
// grad_cost P; cost kind: grad_cost P - that) instead of Gamma.
template <int VEC, int CH>
__global__ __launch_bounds__(kThreads) void unrolled(UnrArgs a) {
    using R = Row<VEC, CH>;
    constexpr int PL = R::PL;
    // LDS: fold (kFoldRows) N | colsum N | v_t N | v_{t-1} N | red N + W | scratch 16
    extern __shared__ float lds[];
    const int wave = threadIdx.x / kWave;
    const int G = gridDim.x;
    const int gid = res::logical_group(a.W);
    const int b = gid / a.W;
    const int w = gid % a.W;
    const int row0 = w * a.R;
    const int rend = min(row0 + a.R, a.M);
    const int c0 = slice_begin(w, a.W, a.N), c1 = slice_begin(w + 1, a.W, a.N);
    float* tree = lds;
    float* lds_cs = tree + kFoldRows<VEC, CH> * a.N;
    float* lds_v = lds_cs + a.N;
    float* lds_vm = lds_v + a.N;
    float* red = lds_vm + a.N;
    float* scratch = red + a.N + a.W;
    const size_t bM = size_t(b) * a.M;
    const bool cost_kind = a.scores_kind < 0;
    const float gc = a.gC ? a.gC[b * a.gc_step] : 0.0f;
    const float csign = cost_kind ? 1.0f : -1.0f;  // C = csign * scores
    bool dead = false;
    float tacc = 0.0f;
    res::announce_xcc(a.part, a.N, b, a.W, w);
    bool local = false;  // set by the XCD check before the first exchange

    // The gradient of a row from its final Gamma (kernels.cu:926-963).
    auto epilogue = [&](size_t off, int ln, float (&gam)[PL], const float (&x)[PL]) {
        float p[PL];
        R::load(a.P + off, ln, a.N, p, 0.0f);
#pragma unroll
        for (int e = 0; e < PL; ++e) {
            const float gl = gam[e] * a.inv_tau;
            const float la = cost_kind ? -x[e] : x[e];
            if (R::valid(ln, e, a.N)) tacc = fmaf(gam[e], la, tacc);
            gam[e] = cost_kind ? gc * p[e] - gl : gl - gc * p[e];
        }
        R::store_stream(a.grad + off, ln, a.N, gam);
    };
    // Column sums of the workgroup's Gamma rows -> every workgroup's lds_cs.
    auto exchange = [&](float (&acc)[PL], unsigned tag) {
        const int cur = tag & 1;
        publish_row<VEC, CH>(acc, tree, a.N, a.part + (size_t(cur) * G + gid) * a.N, tag, local);
        unsigned long long* res_row = a.res + (size_t(cur) * a.B + b) * a.N;
        reduce_slice(a.part + size_t(cur) * G * a.N + size_t(b) * a.W * a.N, a.N, a.W, c0, c1, tag, red,
                     a.spin_limit, a.status, dead, [&](int j, float tot) { publish(res_row + j, tot, tag, local); });
        gather(res_row, a.N, tag, lds_cs, a.spin_limit, a.status, dead);
        __syncthreads();
    };

    // Gamma = G * P (kernels.cu:844-854).
    float acc[PL];
#pragma unroll
    for (int e = 0; e < PL; ++e) acc[e] = 0.0f;
    for (int l = wave; row0 + l < rend; l += kWaves) {
        const size_t off = (bM + row0 + l) * a.N;
        const int ln = opaque_lane();
        float gam[PL], x[PL];
        R::load(a.P + off, ln, a.N, gam, 0.0f);
        R::load(a.X + off, ln, a.N, x, 0.0f);
        if (a.gP) {
            float g[PL];
            R::load(a.gP + off, ln, a.N, g, 0.0f);
#pragma unroll
            for (int e = 0; e < PL; ++e) gam[e] *= g[e] + (a.gC ? gc * (csign * x[e]) : 0.0f);
        } else {
#pragma unroll
            for (int e = 0; e < PL; ++e) gam[e] *= a.gC ? gc * (csign * x[e]) : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < PL; ++e) acc[e] += gam[e];
        if (a.T == 0) epilogue(off, ln, gam, x);
        else R::store(a.gamma + off, ln, a.N, gam);
    }
    local = res::element_on_one_xcd(a.part, a.N, b, a.W, w, a.spin_limit, a.status, dead, scratch) && a.local_ok;
    unsigned tag = 1;
    if (a.T > 0) exchange(acc, tag);

    for (int t = a.T - 1; t >= 0; --t) {
        const float* vt = a.v_hist + (size_t(t) * a.B + b) * a.N;
        const float* vm = t > 0 ? a.v_hist + (size_t(t - 1) * a.B + b) * a.N : nullptr;
        for (int j = threadIdx.x; j < a.N; j += kThreads) {
            lds_v[j] = vt[j];
            lds_vm[j] = vm ? vm[j] : 0.0f;
        }
        __syncthreads();
        const float* ut = a.u_hist + size_t(t) * a.B * a.M + bM;
#pragma unroll
        for (int e = 0; e < PL; ++e) acc[e] = 0.0f;
        for (int l = wave; row0 + l < rend; l += kWaves) {
            const size_t off = (bM + row0 + l) * a.N;
            const int ln = opaque_lane();
            const float ui = ut[row0 + l];
            float gam[PL], x[PL];
            R::load(a.gamma + off, ln, a.N, gam, 0.0f);
            R::load(a.X + off, ln, a.N, x, 0.0f);
            float tl = 0.0f;
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float cs[VEC], vv[VEC];
                R::chunk(lds_cs, ln, k, a.N, cs);
                R::chunk(lds_v, ln, k, a.N, vv);
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    const int e = k * VEC + q;
                    gam[e] = gam[e] - safe_fast_exp((x[e] * a.kscale + ui) + vv[q]) * cs[q];
                    if (R::valid(ln, e, a.N)) tl += gam[e];
                }
            }
            const float ti = wave_sum(tl);
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float vv[VEC];
                R::chunk(lds_vm, ln, k, a.N, vv);
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    const int e = k * VEC + q;
                    gam[e] = gam[e] - safe_fast_exp((x[e] * a.kscale + ui) + vv[q]) * ti;
                    acc[e] += gam[e];
                }
            }
            if (t == 0) epilogue(off, ln, gam, x);
            else R::store(a.gamma + off, ln, a.N, gam);
        }
        if (t > 0) exchange(acc, ++tag);
    }
    const float tsum = block_reduce<kWaves>(wave_sum(tacc), scratch, OpSum{});
    if (threadIdx.x == 0) a.tau_partial[gid] = dead ? __builtin_nanf("") : tsum;
}

// Half rows (32 floats a lane: chunks k = 0 .. HCH - 1 of 256 columns) of a
// [B, M, N] matrix through a buffer resource: one 32-bit offset per row and
// the chunk offsets as constants, so that a row costs one address register
// instead of a 64-bit address per chunk.  `base` is the matrix (at most 2 GiB,
// checked by the launcher).
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t matrix_rsrc(const float* base, size_t floats) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, unsigned(floats * 4), 0x00020000);
}

// x = the half row at byte offset `off` (the lane's first column); columns
// past `nh` (the half's valid width) read as 0 unless FULL.
template <int HCH, bool FULL>
__device__ __forceinline__ void hload(__amdgpu_buffer_rsrc_t r, unsigned off, int lane, int nh, float (&x)[4 * HCH]) {
#pragma unroll
    for (int k = 0; k < HCH; ++k) {
        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, off, k * 1024, 0);
        const bool in = FULL || k * 256 + 4 * lane < nh;
        x[4 * k + 0] = in ? __uint_as_float(t.x) : 0.0f;
        x[4 * k + 1] = in ? __uint_as_float(t.y) : 0.0f;
        x[4 * k + 2] = in ? __uint_as_float(t.z) : 0.0f;
        x[4 * k + 3] = in ? __uint_as_float(t.w) : 0.0f;
    }
}

// Stores the half row's valid columns (aux 2: non-temporal).
template <int HCH, bool FULL, int AUX>
__device__ __forceinline__ void hstore(__amdgpu_buffer_rsrc_t r, unsigned off, int lane, int nh,
                                       const float (&x)[4 * HCH]) {
#pragma unroll
    for (int k = 0; k < HCH; ++k) {
        const u32x4 t = {__float_as_uint(x[4 * k + 0]), __float_as_uint(x[4 * k + 1]), __float_as_uint(x[4 * k + 2]),
                         __float_as_uint(x[4 * k + 3])};
        if (FULL || k * 256 + 4 * lane < nh) __builtin_amdgcn_raw_buffer_store_b128(t, r, off, k * 1024, AUX);
    }
}

// unrolled() for rows of 2049 .. 4096 floats (64 per lane), where Gamma,
// the scores and the column sums of a row would not all fit a lane's
// registers: each row is streamed in two halves of HCH chunks (32 floats per
// lane).  Gamma_Y of both halves and the column sums stay in registers; the
// scores of the half processed first are read again (from the caches) for the
// second update, those of the other half are still in registers.  The
// arithmetic per element, and its order, are unrolled()'s.  FULL: N = 2 HN
// (no partial chunks).
template <int HCH, bool FULL>
__global__ __launch_bounds__(kThreads) void unrolled_halves(UnrArgs a) {
    constexpr int VEC = 4;
    constexpr int CH = 2 * HCH;
    constexpr int HL = VEC * HCH;         // floats per lane per half
    constexpr int HN = HCH * kWave * VEC;  // columns per half
    extern __shared__ float lds[];
    const int wave = threadIdx.x / kWave;
    const int gid = res::logical_group(a.W);
    const int b = gid / a.W;
    const int w = gid % a.W;
    const int row0 = w * a.R;
    const int rend = min(row0 + a.R, a.M);
    const int c0 = slice_begin(w, a.W, a.N), c1 = slice_begin(w + 1, a.W, a.N);
    const int G = gridDim.x;
    float* tree = lds;
    float* lds_cs = tree + kFoldRows<VEC, CH> * a.N;
    float* lds_v = lds_cs + a.N;
    float* lds_vm = lds_v + a.N;
    float* red = lds_vm + a.N;
    float* scratch = red + a.N + a.W;
    const size_t bM = size_t(b) * a.M;
    const size_t total = size_t(a.B) * a.M * a.N;
    const auto rX = matrix_rsrc(a.X, total);
    const auto rG = matrix_rsrc(a.gamma, total);
    const auto rP = matrix_rsrc(a.P, total);
    const auto rGrad = matrix_rsrc(a.grad, total);
    const bool cost_kind = a.scores_kind < 0;
    const float gc = a.gC ? a.gC[b * a.gc_step] : 0.0f;
    const float csign = cost_kind ? 1.0f : -1.0f;  // C = csign * scores
    bool dead = false;
    float tacc = 0.0f;
    res::announce_xcc(a.part, a.N, b, a.W, w);
    bool local = false;  // set by the XCD check before the first exchange
    // byte offset of a lane's first column of half h of row i
    auto offset = [&](int i, int h, int ln) {
        return unsigned((bM + i) * a.N + h * HN) * 4u + unsigned(ln) * 16u;
    };

    // Half h of a row's gradient from its final Gamma (kernels.cu:926-963).
    auto epilogue = [&](unsigned off, int ln, int nh, float (&gam)[HL], const float (&x)[HL]) {
        float p[HL];
        hload<HCH, FULL>(rP, off, ln, nh, p);
#pragma unroll
        for (int e = 0; e < HL; ++e) {
            const float gl = gam[e] * a.inv_tau;
            const float la = cost_kind ? -x[e] : x[e];
            if (FULL || (e / VEC) * 256 + VEC * ln < nh) tacc = fmaf(gam[e], la, tacc);
            gam[e] = cost_kind ? gc * p[e] - gl : gl - gc * p[e];
        }
        hstore<HCH, FULL, 2>(rGrad, off, ln, nh, gam);
    };
    auto exchange = [&](float (&acc)[2 * HL], unsigned tag) {
        const int cur = tag & 1;
        publish_row<VEC, CH>(acc, tree, a.N, a.part + (size_t(cur) * G + gid) * a.N, tag, local);
        unsigned long long* res_row = a.res + (size_t(cur) * a.B + b) * a.N;
        reduce_slice(a.part + size_t(cur) * G * a.N + size_t(b) * a.W * a.N, a.N, a.W, c0, c1, tag, red,
                     a.spin_limit, a.status, dead, [&](int j, float tot) { publish(res_row + j, tot, tag, local); });
        gather(res_row, a.N, tag, lds_cs, a.spin_limit, a.status, dead);
        __syncthreads();
    };

    // Gamma = G * P (kernels.cu:844-854), half by half.
    float acc[2 * HL];
#pragma unroll
    for (int e = 0; e < 2 * HL; ++e) acc[e] = 0.0f;
#pragma unroll 1
    for (int l = wave; row0 + l < rend; l += kWaves) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int ln = opaque_lane();
            const int nh = a.N - h * HN;
            const unsigned off = offset(row0 + l, h, ln);
            float gam[HL], x[HL];
            hload<HCH, FULL>(rP, off, ln, nh, gam);
            hload<HCH, FULL>(rX, off, ln, nh, x);
            if (a.gP) {
                float g[HL];
                hload<HCH, FULL>(matrix_rsrc(a.gP, total), off, ln, nh, g);
#pragma unroll
                for (int e = 0; e < HL; ++e) gam[e] *= g[e] + (a.gC ? gc * (csign * x[e]) : 0.0f);
            } else {
#pragma unroll
                for (int e = 0; e < HL; ++e) gam[e] *= a.gC ? gc * (csign * x[e]) : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < HL; ++e) acc[h * HL + e] += gam[e];
            if (a.T == 0) epilogue(off, ln, nh, gam, x);
            else hstore<HCH, FULL, 0>(rG, off, ln, nh, gam);
        }
    }
    local = res::element_on_one_xcd(a.part, a.N, b, a.W, w, a.spin_limit, a.status, dead, scratch) && a.local_ok;
    unsigned tag = 1;
    if (a.T > 0) exchange(acc, tag);

    for (int t = a.T - 1; t >= 0; --t) {
        const float* vt = a.v_hist + (size_t(t) * a.B + b) * a.N;
        const float* vm = t > 0 ? a.v_hist + (size_t(t - 1) * a.B + b) * a.N : nullptr;
        for (int j = threadIdx.x; j < a.N; j += kThreads) {
            lds_v[j] = vt[j];
            lds_vm[j] = vm ? vm[j] : 0.0f;
        }
        __syncthreads();
        const float* ut = a.u_hist + size_t(t) * a.B * a.M + bM;
#pragma unroll
        for (int e = 0; e < 2 * HL; ++e) acc[e] = 0.0f;
#pragma unroll 1
        for (int l = wave; row0 + l < rend; l += kWaves) {
            // u_t of the row: wave-uniform, read through the scalar unit (this
            // kernel does not write u_hist)
            const float ui = *(const __attribute__((address_space(4))) float*)(reinterpret_cast<uintptr_t>(ut + row0 + l));
            float gy[2 * HL];  // Gamma_Y of the row
            float x[HL];       // the scores of the half processed last
            float tl = 0.0f;
            // Gamma_Y = Gamma - safe_exp(K + u_t + v_t) colsum(Gamma), and its row sum
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int ln = opaque_lane();
                const int nh = a.N - h * HN;
                const unsigned off = offset(row0 + l, h, ln);
                float gam[HL];
                hload<HCH, FULL>(rG, off, ln, nh, gam);
                hload<HCH, FULL>(rX, off, ln, nh, x);
#pragma unroll
                for (int k = 0; k < HCH; ++k) {
                    float cs[VEC], vv[VEC];
                    const int c = h * HN + k * 256 + VEC * ln;
                    const float4 cs4 = *reinterpret_cast<const float4*>(lds_cs + min(c, a.N - VEC));
                    const float4 vv4 = *reinterpret_cast<const float4*>(lds_v + min(c, a.N - VEC));
                    cs[0] = cs4.x; cs[1] = cs4.y; cs[2] = cs4.z; cs[3] = cs4.w;
                    vv[0] = vv4.x; vv[1] = vv4.y; vv[2] = vv4.z; vv[3] = vv4.w;
                    const bool in = FULL || k * 256 + VEC * ln < nh;
#pragma unroll
                    for (int q = 0; q < VEC; ++q) {
                        const int e = k * VEC + q;
                        const float y = gam[e] - safe_fast_exp((x[e] * a.kscale + ui) + vv[q]) * (in ? cs[q] : 0.0f);
                        gy[h * HL + e] = y;
                        if (in) tl += y;
                    }
                }
            }
            const float ti = wave_sum(tl);
            // Gamma = Gamma_Y - safe_exp(K + u_t + v_{t-1}) rowsum(Gamma_Y): the
            // second half first (its scores are in registers), then the first
            // half with its scores read again
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int h = 1 - hh;
                const int ln = opaque_lane();
                const int nh = a.N - h * HN;
                const unsigned off = offset(row0 + l, h, ln);
                if (h == 0) hload<HCH, FULL>(rX, off, ln, nh, x);
                float gam[HL];
#pragma unroll
                for (int k = 0; k < HCH; ++k) {
                    float vv[VEC];
                    const int c = h * HN + k * 256 + VEC * ln;
                    const float4 vv4 = *reinterpret_cast<const float4*>(lds_vm + min(c, a.N - VEC));
                    vv[0] = vv4.x; vv[1] = vv4.y; vv[2] = vv4.z; vv[3] = vv4.w;
#pragma unroll
                    for (int q = 0; q < VEC; ++q) {
                        const int e = k * VEC + q;
                        gam[e] = gy[h * HL + e] - safe_fast_exp((x[e] * a.kscale + ui) + vv[q]) * ti;
                        acc[h * HL + e] += gam[e];
                    }
                }
                if (t == 0) epilogue(off, ln, nh, gam, x);
                else hstore<HCH, FULL, 0>(rG, off, ln, nh, gam);
            }
        }
        if (t > 0) exchange(acc, ++tag);
    }
    const float tsum = block_reduce<kWaves>(wave_sum(tacc), scratch, OpSum{});
    if (threadIdx.x == 0) a.tau_partial[gid] = dead ? __builtin_nanf("") : tsum;
}

}  // namespace pst
}  // namespace dot_amd
