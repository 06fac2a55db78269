// Register-resident persistent kernels.
//
// When one batch element's [M, N] matrix fits the vector registers of W
// workgroups (8 waves each, one workgroup per CU), the iterations run inside
// one cooperative launch: every workgroup loads its strip of rows into VGPRs
// once and then only exchanges one row of per-column partial sums per
// iteration with the other W-1 workgroups of its batch element.
//
// Exchange protocol.  Cross-workgroup agent-scope release/acquire fences
// write back and invalidate the per-XCD L2 and serialise across workgroups,
// which costs more than a kernel launch on MI355X.  Instead every exchanged
// value travels with its iteration number: a 64-bit word (float bits low,
// iteration tag high) written and read with relaxed agent-scope atomics,
// which are single-copy atomic and coherent per location.  A reader polls
// until the tag it expects appears, so no separate flag or fence is needed.
// Slots alternate by iteration parity, which keeps a fast workgroup from
// overwriting a slot before the slow ones have read it (it cannot finish
// iteration t+1 before everyone has published iteration t+1, which each
// workgroup does only after reading iteration t).  Polls are bounded; a
// timeout sets `status` and the outputs are written as NaN.
#pragma once

#include <cfloat>
#include <cstdint>

#include "row.cuh"
#include "sinkhorn_kernels.cuh"

namespace dot_amd {
namespace res {

// 8 waves per workgroup (2 per SIMD) leave each wave 256 registers, of which
// up to 128 per lane hold the resident strip; a 16-wave workgroup would hold
// the same strip in 64 registers per lane but leave only 64 for everything else.
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;  // 8
constexpr int kMaxRegFloats = 128;        // per-lane VGPR budget for the resident strip
constexpr int kMaxGroup = 8;              // workgroups per batch element (staging rows in LDS)

__device__ __forceinline__ unsigned long long tag_pack(float v, unsigned t) {
    return (static_cast<unsigned long long>(t) << 32) | __float_as_uint(v);
}

__device__ __forceinline__ void publish(unsigned long long* p, float v, unsigned t) {
    __hip_atomic_store(p, tag_pack(v, t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exchange words read only by workgroups on the writer's XCD.  An agent-scope
// store writes through to memory; a workgroup-scope store stops in the XCD's
// L2 (the vector L1 is write-through), where the readers' agent-scope loads
// find it: a tagged ping-pong between two workgroups of one XCD takes 0.53 us
// per round trip this way against 1.09 us with agent-scope stores.  A word
// stored this way is not visible to another XCD before its line leaves the
// L2, so `local` must be true only when every reader runs on the writer's XCD
// (element_on_one_xcd).
__device__ __forceinline__ void publish(unsigned long long* p, float v, unsigned t, bool local) {
    if (local)
        __hip_atomic_store(p, tag_pack(v, t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
        __hip_atomic_store(p, tag_pack(v, t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The XCD (XCC) this workgroup runs on.
__device__ __forceinline__ int xcc_id() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return int(x & 0xfu);
}

// Waits for slot `p` to carry tag `t` and returns its value.  Gives up after
// `spin_limit` polls, or as soon as any workgroup has reported a timeout in
// `status` (checked every 256 polls); `dead` then short-circuits every later
// call of this lane, so a failure costs one bounded wait, not one per value.
//
// `mark` is this call's failure mark: a wait that gives up raises the status
// word to it (atomic max), and a status at or above it means this call has
// failed.  A status word cleared for the call takes mark 1; one that persists
// across calls takes marks that grow from call to call (the call epoch).
__device__ __forceinline__ void forced_timeout(int spin_limit, int* status, bool& dead, int mark = 1) {
    // A negative limit (set by the host only to test the error path) makes
    // every bounded wait give up at once, without polling.
    if (spin_limit < 0 && !dead) {
        atomicMax(status, mark);
        dead = true;
    }
}

__device__ __forceinline__ float collect(unsigned long long* p, unsigned t, int spin_limit,
                                         int* status, bool& dead, int mark = 1) {
    forced_timeout(spin_limit, status, dead, mark);
    if (dead) return __builtin_nanf("");
    for (int spins = 0;; ++spins) {
        const unsigned long long x = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (static_cast<unsigned>(x >> 32) == t) return __uint_as_float(static_cast<unsigned>(x));
        if ((spins & 255) == 255 &&
            __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= mark) {
            dead = true;
            return __builtin_nanf("");
        }
        if (spins >= spin_limit) {
            atomicMax(status, mark);
            dead = true;
            return __builtin_nanf("");
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Tag of the XCD-id words in slots cleared for the call, whose exchange tags
// are iteration numbers (>= 1), so this one never matches them.  Slots that
// persist across calls carry (epoch << 16) | t, and (epoch << 16) | 0xffff for
// the XCD ids (callers pass `tag`).
constexpr unsigned kXccTag = 0xfffffffeu;

// Tag of the per-workgroup result words (partial sums and failure flags
// published once, at the end of a launch) in slots cleared for the call; an
// iteration tag reaches it only past 2^32 - 4 iterations.  Slots that persist
// across calls use (epoch << 16) | 0xfffe, above every tagged iteration.
constexpr unsigned kResultTag = 0xfffffffdu;

// The sum over batch element b's W workgroups of one value each, added in the
// order w = 0, 1, ... by workgroup 0 of the element, which waits for the
// other W - 1 in `words` (one per logical workgroup gid = b * W + w) and
// returns the sum; the others publish theirs and return 0.  Thread 0 only.
__device__ __forceinline__ float element_sum(unsigned long long* words, int gid, int w, int W, float mine,
                                             unsigned tag, int spin_limit, int* status, bool& dead, int mark) {
    if (w != 0) {
        publish(words + gid, mine, tag);
        return 0.0f;
    }
    float s = mine;
    for (int q = 1; q < W; ++q) s += collect(words + gid + q, tag, spin_limit, status, dead, mark);
    return s;
}

// Whether any workgroup of the grid failed (a wait that gave up, or the
// status word at the call's failure mark): every workgroup publishes its
// flag `bad` to words[gid] and logical workgroup 0 waits for all G flags (a
// wait for one that gives up counts as a failure).  Returns the verdict in
// every thread of workgroup 0, and false elsewhere.  Every thread must call it.
__device__ __forceinline__ bool grid_failed(unsigned long long* words, int gid, int G, bool bad, unsigned tag,
                                            int spin_limit, int* status, bool& dead, int mark) {
    if (threadIdx.x == 0) publish(words + gid, bad ? 1.0f : 0.0f, tag);
    if (gid != 0) return false;
    int any = 0;
    for (int g = threadIdx.x; g < G; g += blockDim.x)
        any |= collect(words + g, tag, spin_limit, status, dead, mark) != 0.0f;  // NaN: gave up
    return __syncthreads_or(any) != 0;
}

// XCD check of a batch element, in two steps so that the round trip hides
// under other work.  announce_xcc: each workgroup publishes its XCC id (agent
// scope) into word 0 of its row `rows + (b * W + w) * stride`.  The row must
// be one that no workgroup of the element writes again before every
// workgroup of the element has passed element_on_one_xcd (the sweep slot of
// iteration parity 0 qualifies: iteration 2 is published only after every
// workgroup has published iteration 1, which each does after the check).
__device__ __forceinline__ void announce_xcc(unsigned long long* rows, size_t stride, int b, int W, int w,
                                             unsigned tag = kXccTag) {
    if (threadIdx.x == 0) publish(rows + (size_t(b) * W + w) * stride, __int_as_float(xcc_id()), tag);
}

// True when the W workgroups of batch element b (this one is w) all run on
// one XCD, so that their exchanges may use publish(..., local = true): wave 0
// reads the element's W announced ids.  A timeout reads as "not one XCD" (and
// sets `dead` as any poll does).  Contains barriers; every thread must call it.
__device__ __forceinline__ bool element_on_one_xcd(unsigned long long* rows, size_t stride, int b, int W, int w,
                                                   int spin_limit, int* status, bool& dead, float* scratch,
                                                   unsigned tag = kXccTag, int mark = 1) {
    const int me = xcc_id();
    if (threadIdx.x < kWave) {
        const int g = threadIdx.x;
        int same = 1;
        if (g < W && g != w)
            same = __float_as_int(collect(rows + (size_t(b) * W + g) * stride, tag, spin_limit, status,
                                          dead, mark)) == me;
        const int all = __all(same);
        if (g == 0) scratch[0] = all ? 1.0f : 0.0f;
    }
    __syncthreads();
    const bool local = scratch[0] != 0.0f;
    __syncthreads();
    return local;
}

// Collects one published row (this lane's PL columns) with every load of a poll
// round in flight at once; returns false after a timeout (values are then NaN).
template <int VEC, int CH>
__device__ __forceinline__ void collect_row(unsigned long long* row, unsigned t, int N, int spin_limit,
                                            int* status, bool& dead, float (&out)[VEC * CH], int mark) {
    using R = Row<VEC, CH>;
    const int lane = threadIdx.x % kWave;
    forced_timeout(spin_limit, status, dead, mark);
    if (dead) {
#pragma unroll
        for (int e = 0; e < R::PL; ++e) out[e] = __builtin_nanf("");
        return;
    }
    for (int spins = 0;; ++spins) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < CH; ++k) {
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                const int col = R::col(lane, k) + v;
                unsigned long long x = tag_pack(0.0f, t);
                if (col < N) x = __hip_atomic_load(row + col, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ready = ready && static_cast<unsigned>(x >> 32) == t;
                out[k * VEC + v] = __uint_as_float(static_cast<unsigned>(x));
            }
        }
        if (ready) return;
        if (((spins & 255) == 255 &&
             __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= mark) ||
            spins >= spin_limit) {
            if (spins >= spin_limit) atomicMax(status, mark);
            dead = true;
#pragma unroll
            for (int e = 0; e < R::PL; ++e) out[e] = __builtin_nanf("");
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Fold the waves' per-lane column values into wave 0 in a fixed order
// (halving tree 4, 2, 1).  `lds` holds kWaves/2 * N floats.  Every thread must call it.
template <int VEC, int CH, class Op = OpSum>
__device__ __forceinline__ void tree_combine(float (&acc)[VEC * CH], float* lds, int N, Op op = Op{}) {
    using R = Row<VEC, CH>;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
#pragma unroll
    for (int half = kWaves / 2; half >= 1; half /= 2) {
        __syncthreads();
        if (wave >= half && wave < 2 * half) R::store(lds + (wave - half) * N, lane, N, acc);
        __syncthreads();
        if (wave < half) {
            float o[R::PL];
            R::load(lds + wave * N, lane, N, o, 0.0f);
#pragma unroll
            for (int e = 0; e < R::PL; ++e) acc[e] = op(acc[e], o[e]);
        }
    }
}

// Lane exchange across the two 32-lane halves (lane ^ 32).
__device__ __forceinline__ float xor32(float x) {
    const int lane = threadIdx.x % kWave;
    return __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, x)));
}

// Partner patterns of the transposed reduction, in the order they are used:
// row mirror (lane ^ 15), half-row mirror (lane ^ 7), quad xor 2, quad xor 1.
// Each flips the lane bit that step s selects on (3 - s) and none of the
// bits selected on by earlier steps, so partners always hold the same rows.
template <int S>
__device__ __forceinline__ float tstep_move(float x) {
    if constexpr (S == 0) return dpp_move<kDppRowMirror>(x);
    else if constexpr (S == 1) return dpp_move<kDppRowHalfMirror>(x);
    else if constexpr (S == 2) return dpp_move<kDppQuadXor2>(x);
    else return dpp_move<kDppQuadXor1>(x);
}

constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x / 2); }

template <int N, int S, class Op>
__device__ __forceinline__ float treduce_level(const float* v, int lane, Op op) {
    if constexpr (N == 1) {
        float x = v[0];
        if constexpr (S <= 0) x = op(x, tstep_move<0>(x));
        if constexpr (S <= 1) x = op(x, tstep_move<1>(x));
        if constexpr (S <= 2) x = op(x, tstep_move<2>(x));
        if constexpr (S <= 3) x = op(x, tstep_move<3>(x));
        x = op(x, swizzle_xor16(x));
        return op(x, xor32(x));
    } else {
        constexpr int H = N / 2;
        const bool upper = (lane >> (3 - S)) & 1;
        float w[H];
#pragma unroll
        for (int j = 0; j < H; ++j) {
            const float keep = upper ? v[j + H] : v[j];
            const float send = upper ? v[j] : v[j + H];
            w[j] = op(keep, tstep_move<S>(send));
        }
        return treduce_level<H, S + 1>(w, lane, op);
    }
}

// Wave reductions of RPW per-lane values at once (RPW a power of two <= 16):
// at each butterfly step the two partner lanes trade halves of their
// remaining rows, so step s moves RPW / 2^(s+1) values instead of RPW.  Every
// lane returns the wave total of row slot_of_lane(lane); the four lanes that
// share a slot return the same bits.
template <int RPW, class Op>
__device__ __forceinline__ float transposed_reduce(const float (&v)[RPW], Op op) {
    static_assert(RPW >= 1 && RPW <= 16 && (RPW & (RPW - 1)) == 0, "RPW must be 1, 2, 4, 8 or 16");
    return treduce_level<RPW, 0>(v, threadIdx.x % kWave, op);
}

template <int RPW>
__device__ __forceinline__ float transposed_sum(const float (&v)[RPW]) {
    return transposed_reduce<RPW>(v, OpSum{});
}

template <int RPW>
__device__ __forceinline__ int slot_of_lane(int lane) {
    return (lane & 15) >> (4 - ilog2(RPW));
}

template <int RPW>
__device__ __forceinline__ int lane_of_slot(int k) {
    return k << (4 - ilog2(RPW));
}

constexpr int kColsPerThread = (1024 + kThreads - 1) / kThreads;  // N <= 1024

// Column rounds of the per-column exchange for rows of PL floats per lane
// (64 PL columns at most): thread t takes columns t, t + kThreads, ...
template <int PL>
constexpr int kColRounds = (kWave * PL + kThreads - 1) / kThreads;
constexpr int kXcds = 8;  // MI355X dispatches consecutive workgroups round-robin over 8 XCDs

// Logical index of this workgroup, b * W + w.  When the grid splits evenly,
// the W workgroups of a batch element are given blocks on one XCD, where an
// exchange round trip is ~0.9 us instead of ~1.25 us; any bijection is correct.
__device__ __forceinline__ int logical_group(int W) {
    const int G = gridDim.x;
    const int per = G / kXcds;
    if (G % kXcds == 0 && per % W == 0) return (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
    return blockIdx.x;
}

// Element q of a small per-thread array through static indices only (a
// dynamic index would place the array in scratch memory, and every reload
// from there waits for all memory operations in flight).
template <int N>
__device__ __forceinline__ float pick(const float (&v)[N], int q) {
    float r = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i)
        if (q == i) r = v[i];
    return r;
}
template <int N>
__device__ __forceinline__ void put(float (&v)[N], int q, float x) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (q == i) v[i] = x;
}

// Batch-element column totals for this thread's columns j = tid + q*kThreads.
// `part` holds one row of N per wave; the workgroup's sum of column j is the
// sum of those rows in wave order, published with tag t into slot row `gid`
// (= b * W + w); the total adds the W workgroups' sums of the element in
// workgroup order (every workgroup of the element gets the same bits).
// Every lane polls its own values (a separate "ready" word would add a
// second memory round trip).  f(j, total) consumes each total; totals are
// NaN after a timeout.  `local`: every workgroup of the element runs on this
// XCD (element_on_one_xcd).  NQ: column rounds (kColRounds of the row layout).
// MG >= W: the workgroups per element the poll registers are sized for (an
// element of at most 4 workgroups polls from half the registers).
template <int NQ, int MG = kMaxGroup, class F>
__device__ __forceinline__ void exchange_columns(const float* part, unsigned long long* slot, int N,
                                                 int b, int W, int w, unsigned t, bool local, int spin_limit,
                                                 int* status, bool& dead, int mark, F&& f) {
    static_assert(NQ >= 1 && NQ <= kColsPerThread, "rows of at most 1024 columns");
    static_assert(MG >= 1 && MG <= kMaxGroup, "at most kMaxGroup workgroups per element");
    float own[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int j = threadIdx.x + q * kThreads;
        own[q] = 0.0f;
        if (j < N) {
            float s = 0.0f;
#pragma unroll
            for (int v = 0; v < kWaves; ++v) s += part[v * N + j];
            own[q] = s;
            if (W > 1) publish(slot + (size_t(b) * W + w) * N + j, s, t, local);
        }
    }
    unsigned long long* base = slot + size_t(b) * W * N;
    forced_timeout(spin_limit, status, dead, mark);
    // The guards below depend only on the thread and the element; computed
    // from these opaque copies they are rebuilt at each call instead of being
    // hoisted out of the caller's iteration loop and held in scalar registers
    // for the whole kernel (C3 adjoint: 70 -> 42 spilled SGPRs, 3 % faster).
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    asm volatile("" : "+s"(W), "+s"(w));
    // One poll round issues the loads of every (column, workgroup) pair first
    // and only then looks at the tags, so the round costs one memory latency
    // (a load whose tag is tested before the next load is issued makes the
    // compiler wait for each in turn).  Pairs outside the element or the row,
    // and this workgroup's own slot, are not loaded and count as ready.
    float got[NQ][MG] = {};
    for (int spins = 0; W > 1 && !dead; ++spins) {
        unsigned long long x[NQ][MG];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int j = tid + q * kThreads;
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                x[q][g] = tag_pack(0.0f, t);
                if (g < W && g != w && j < N)
                    x[q][g] = __hip_atomic_load(base + size_t(g) * N + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        bool ready = true;
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                ready = ready && static_cast<unsigned>(x[q][g] >> 32) == t;
                got[q][g] = __uint_as_float(static_cast<unsigned>(x[q][g]));
            }
        if (ready) break;
        if (((spins & 255) == 255 &&
             __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= mark) ||
            spins >= spin_limit) {
            if (spins >= spin_limit) atomicMax(status, mark);
            dead = true;
            break;
        }
        // Rounds go back to back: a round is one memory latency (~0.6 us under
        // the sweep's load at C3), and a 64-clock sleep between rounds cost
        // 0.05 us per sweep; issuing the next round before testing the last
        // one (two in flight) cost 0.15 us.
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int j = threadIdx.x + q * kThreads;
        if (j >= N) continue;
        const float mine = own[q];
        float tot = 0.0f;
#pragma unroll
        for (int g = 0; g < MG; ++g)
            if (g < W) tot += (g == w) ? mine : got[q][g];
        f(j, dead ? __builtin_nanf("") : tot);
    }
}

struct ImpResArgs {
    const float* X;            // scores
    int scores_kind;
    const float* gP;           // [B,M,N] or null
    const float* gC;           // [B] or null
    int gc_step;               // 1, or 0: gC holds one value for every batch element
    const float* P;            // [B,M,N]
    unsigned long long* xchg;  // [2, G, N] tagged sweep column sums
    unsigned long long* pro;   // [2, G, N] tagged prologue column sums (P G, then P)
    float* grad;               // [B,M,N]
    float* grad_tau;           // [B] out: tau_scale * sum(grad * log_alpha)
    float tau_scale;
    unsigned long long* rwords;  // [2, G] tagged result words: grad_tau partials, failure flags
    unsigned result_tag;
    int32_t* status_out;       // the caller's status word (1: a wait gave up), or null
    int keep_status;           // nonzero: raise status_out only (a later slab of one call)
    int* status;
    float inv_tau;
    int M, N, W, R, iters, spin_limit;
    unsigned tag_base;         // exchange tags are tag_base | t (0: slots cleared for the call)
    unsigned xcc_tag;          // tag of the XCD-id words
    int mark;                  // failure mark in *status (forced_timeout)
    int32_t* sweeps;           // [B] sweeps executed per batch element, or null
    int early;                 // nonzero: end each element's sweeps once converged (sk::AdjointStop)
    int local_ok;              // XCD-local exchange stores allowed (local_exchange_allowed)
};

// Upstream gradient of one row: G = grad_plan + grad_cost[b] * C, C = csign * scores.
template <int VEC, int CH>
__device__ __forceinline__ void upstream_row(const ImpResArgs& a, size_t off, int lane, float gc,
                                             float csign, float (&x)[VEC * CH], float (&G)[VEC * CH]) {
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

// The implicit adjoint (kernels.cu:965-1098) with P held in registers, in one
// launch.  Prologue: r_i = sum_k P G, rs_i = sum_k P for this workgroup's rows
// and, through one exchange each, c_k = sum_i P G and cs_k = sum_i P over the
// batch element.  Each of the `iters` Gauss-Seidel sweeps (from lambda = mu = 0):
//   lambda_i = (r_i - sum_k P mu_k) / max(rs_i, 1e-12)   (all rows of a wave at once)
//   mu_k = (c_k - sum_i P lambda_i) / max(cs_k, 1e-12)   (one exchange)
// Final phase: grad = P (G - lambda - mu) / tau (cost kind: grad_cost P - that;
// log-alpha kind: that - grad_cost P) and this workgroup's share of
// sum(grad * log_alpha), which workgroup 0 of the element adds up into
// grad_tau; with status_out, logical workgroup 0 also writes the call's
// status word once every workgroup has reported.  MG >= W (exchange_columns).
// With `early`, an element's sweeps end once sk::AdjointStop finds them
// converged.
template <int VEC, int CH, int RPW, int MG = kMaxGroup>
__global__ __launch_bounds__(kThreads) void implicit_adjoint(ImpResArgs a) {
    using R = Row<VEC, CH>;
    constexpr int PL = R::PL;
    // LDS: one row of N per wave | mu N | scratch kWaves | per-wave values of the stop test 2 kWaves
    extern __shared__ float lds[];
    float* part = lds;
    float* lds_mu = lds + kWaves * a.N;
    float* scratch = lds_mu + a.N;
    float* stopbuf = scratch + kWaves;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int G = gridDim.x;
    const int gid = logical_group(a.W);
    const int b = gid / a.W;
    const int w = gid % a.W;
    const int row0 = w * a.R;
    const int rend = min(row0 + a.R, a.M);
    const size_t bM = size_t(b) * a.M;
    const bool cost_kind = a.scores_kind < 0;
    const float gc = a.gC ? a.gC[b * a.gc_step] : 0.0f;
    const float csign = cost_kind ? 1.0f : -1.0f;  // C = csign * scores
    bool dead = false;
    announce_xcc(a.xchg, a.N, b, a.W, w, a.xcc_tag);

    // The strip of P, loaded once into the registers it stays in for every sweep.
    float p[RPW][PL];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        const int i = row0 + wave + kWaves * k;
        if (i < rend) {
            R::load(a.P + (bM + i) * a.N, lane, a.N, p[k], 0.0f);
        } else {
#pragma unroll
            for (int e = 0; e < PL; ++e) p[k][e] = 0.0f;
        }
    }
    // Prologue, from the registers with G streamed row by row: row sums
    // r = sum_k P G and rs = sum_k P of this wave's rows (reduced across the
    // wave together, each lane keeping one row's, as the sweeps' row dots) and
    // the workgroup's column partials of P G and P.
    float cg[PL], cp[PL], sg[RPW], sp[RPW];
#pragma unroll
    for (int e = 0; e < PL; ++e) cg[e] = cp[e] = 0.0f;
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        sg[k] = sp[k] = 0.0f;
        const int i = row0 + wave + kWaves * k;
        if (i < rend) {
            float x[PL], Gr[PL];
            upstream_row<VEC, CH>(a, (bM + i) * a.N, lane, gc, csign, x, Gr);
#pragma unroll
            for (int e = 0; e < PL; ++e) {
                sg[k] = fmaf(p[k][e], Gr[e], sg[k]);
                sp[k] += p[k][e];
                cg[e] = fmaf(p[k][e], Gr[e], cg[e]);
                cp[e] += p[k][e];
            }
        }
    }
    const float r_l = transposed_sum<RPW>(sg);
    const float rs_l = transposed_sum<RPW>(sp);
    const float inv_rs = 1.0f / fmaxf(rs_l, sk::kSumFloor);
    float c_own[kColRounds<PL>], cs_own[kColRounds<PL>];
    const bool local =
        element_on_one_xcd(a.xchg, a.N, b, a.W, w, a.spin_limit, a.status, dead, scratch, a.xcc_tag, a.mark) &&
        a.local_ok;
    R::store(part + wave * a.N, lane, a.N, cg);
    __syncthreads();
    exchange_columns<kColRounds<PL>, MG>(part, a.pro, a.N, b, a.W, w, a.tag_base | 1u, local, a.spin_limit,
                                         a.status, dead, a.mark,
                                         [&](int j, float tot) { put(c_own, (j - threadIdx.x) / kThreads, tot); });
    __syncthreads();
    R::store(part + wave * a.N, lane, a.N, cp);
    __syncthreads();
    exchange_columns<kColRounds<PL>, MG>(part, a.pro + size_t(G) * a.N, a.N, b, a.W, w, a.tag_base | 1u, local,
                                         a.spin_limit, a.status, dead, a.mark, [&](int j, float tot) {
                                         put(cs_own, (j - threadIdx.x) / kThreads, fmaxf(tot, sk::kSumFloor));
                                     });

    // Sweeps, from mu = 0.  Thread j % kThreads writes (and reads back) column j of
    // lds_mu in exchange_columns' callback, so its own zeroing needs no barrier.
    float mu[PL];
#pragma unroll
    for (int e = 0; e < PL; ++e) mu[e] = 0.0f;
    for (int j = threadIdx.x; j < a.N; j += kThreads) lds_mu[j] = 0.0f;
    float lam_l = 0.0f;
    sk::AdjointStop stop;
    int done_t = a.iters;
    for (int t = 1; t <= a.iters; ++t) {
        float d[RPW];  // one dependent chain per row; the rows give the parallelism
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            d[k] = 0.0f;
#pragma unroll
            for (int e = 0; e < PL; ++e) d[k] = fmaf(p[k][e], mu[e], d[k]);
        }
        lam_l = (r_l - transposed_sum<RPW>(d)) * inv_rs;
        float acc[PL];
#pragma unroll
        for (int e = 0; e < PL; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            const float lk = read_lane(lam_l, lane_of_slot<RPW>(k));
#pragma unroll
            for (int e = 0; e < PL; ++e) acc[e] = fmaf(p[k][e], lk, acc[e]);
        }
        // No barrier needed here: the last readers of part and lds_mu (the
        // previous exchange and mu reload) are behind the barrier that ends
        // the previous sweep.
        R::store(part + wave * a.N, lane, a.N, acc);
        __syncthreads();
        // this thread's largest |mu_t - mu_{t-1}| and (|c_k| + |sum_i P lambda_i|) / cs_k
        float dmu = 0.0f, smu = 0.0f;
        exchange_columns<kColRounds<PL>, MG>(part, a.xchg + size_t(t & 1) * G * a.N, a.N, b, a.W, w,
                                             a.tag_base | unsigned(t), local, a.spin_limit, a.status, dead,
                                             a.mark, [&](int j, float tot) {
                                             const int q = (j - threadIdx.x) / kThreads;
                                             const float cj = pick(c_own, q), csj = pick(cs_own, q);
                                             const float m = (cj - tot) / csj;
                                             dmu = fmaxf(dmu, fabsf(m - lds_mu[j]));
                                             smu = fmaxf(smu, (fabsf(cj) + fabsf(tot)) / csj);
                                             lds_mu[j] = m;
                                         });
        if (a.early) {
            dmu = wave_max(dmu);
            smu = wave_max(smu);
            if (lane == 0) {
                stopbuf[wave] = dmu;
                stopbuf[kWaves + wave] = smu;
            }
        }
        __syncthreads();
        R::load(lds_mu, lane, a.N, mu, 0.0f);
        if (a.early && t < a.iters) {
            // The last readers of stopbuf are behind the barrier before the next exchange.
            float d = stopbuf[0], sm = stopbuf[kWaves];
#pragma unroll
            for (int q = 1; q < kWaves; ++q) {
                d = fmaxf(d, stopbuf[q]);
                sm = fmaxf(sm, stopbuf[kWaves + q]);
            }
            if (stop.done(t, d, sm)) {
                done_t = t;
                break;
            }
        }
    }
    if (a.sweeps && w == 0 && threadIdx.x == 0) a.sweeps[b] = done_t;

    // Final phase: stream G again and write this workgroup's gradient rows.
    const bool failed = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= a.mark;
    float tacc = 0.0f;
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        const int i = row0 + wave + kWaves * k;
        const float lam = read_lane(lam_l, lane_of_slot<RPW>(k));
        if (i >= rend) continue;
        const size_t off = (bM + i) * a.N;
        float x[PL], Gr[PL], o[PL];
        upstream_row<VEC, CH>(a, off, lane, gc, csign, x, Gr);
#pragma unroll
        for (int e = 0; e < PL; ++e) {
            const float gl = (p[k][e] * ((Gr[e] - lam) - mu[e])) * a.inv_tau;
            const float la = cost_kind ? -x[e] : x[e];
            if (R::valid(lane, e, a.N)) tacc = fmaf(gl, la, tacc);
            o[e] = failed ? __builtin_nanf("") : (cost_kind ? gc * p[k][e] - gl : gl - gc * p[k][e]);
        }
        R::store_stream(a.grad + off, lane, a.N, o);
    }
    const float tsum = block_reduce<kWaves>(wave_sum(tacc), scratch, OpSum{});
    if (threadIdx.x == 0) {
        const float s = element_sum(a.rwords, gid, w, a.W, failed ? __builtin_nanf("") : tsum, a.result_tag,
                                    a.spin_limit, a.status, dead, a.mark);
        if (w == 0) a.grad_tau[b] = s * a.tau_scale;
    }
    if (a.status_out) {
        const bool bad = __syncthreads_or(dead) != 0 || failed;
        const bool any = grid_failed(a.rwords + G, gid, G, bad, a.result_tag, a.spin_limit, a.status, dead,
                                     a.mark);
        if (gid == 0 && threadIdx.x == 0) {
            if (any) *a.status_out = 1;
            else if (!a.keep_status) *a.status_out = 0;
        }
    }
}

}  // namespace res
}  // namespace dot_amd

namespace dot_amd {
namespace res {

constexpr int kDeltaSlots = 4;  // lagged stop test: workgroups drift at most 2 iterations apart
constexpr int kFwdScratch = 32;

struct OpMaxNan {  // max that keeps a NaN (a timed-out poll) instead of dropping it
    __device__ __forceinline__ float operator()(float a, float b) const {
        return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
    }
};

struct FwdResArgs {
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
    float* cost;          // [B] out: sum(P C), or null
    unsigned long long* cwords;  // [G] tagged cost partials of the workgroups
    unsigned result_tag;
    float* u_out;         // [B,M] or null
    float* v_out;         // [B,N] or null
    float* u_hist;        // [T,B,M] or null
    float* v_hist;        // [T,B,N] or null
    int32_t* iters_used;
    int32_t* converged;
    unsigned long long* xchg;   // [2, G, N] tagged column partials
    unsigned long long* fxchg;  // [2, 2, G, N] tagged exact-fallback column max / sum
    unsigned long long* dxchg;  // [kDeltaSlots, G] tagged per-workgroup deltas
    int* status;                // at least `mark` after a poll timeout of this call
    int B, M, N, W, R, spin_limit;
    unsigned tag_base;          // exchange tags are tag_base | t (0: slots cleared for the call)
    unsigned xcc_tag;           // tag of the XCD-id words
    int mark;                   // failure mark in *status (forced_timeout)
    int local_ok;               // XCD-local exchange stores allowed (local_exchange_allowed)
    int lagged_shift;           // shift the row exponentials by the last iteration's LSE
};

// Waits for G tagged per-workgroup deltas of iteration t and returns their
// maximum (order-free, so every workgroup gets the same value).  Every thread
// must call it; wave 0 polls.
__device__ __forceinline__ float global_delta(const FwdResArgs& a, int t, float* scratch, bool& dead) {
    const int lane = threadIdx.x % kWave;
    const int G = gridDim.x;
    __syncthreads();
    if (threadIdx.x < kWave) {
        unsigned long long* ds = a.dxchg + size_t(t % kDeltaSlots) * G;
        float m = 0.0f;
        for (int g = lane; g < G; g += kWave) {
            const float d = collect(ds + g, a.tag_base | unsigned(t), a.spin_limit, a.status, dead, a.mark);
            m = (d != d) ? d : fmaxf(m, d);  // NaN (timeout) propagates
        }
        m = wave_reduce(m, OpMaxNan{});
        if (lane == 0) scratch[0] = m;
    }
    __syncthreads();
    return scratch[0];
}

// Dual log-domain Sinkhorn forward (torch_cuda.cpp:147-264) with the scores
// of this workgroup's rows held in registers for all iterations.
// Iteration t: the row update of sk::fwd_sweep from v_{t-1}, whose shared
// exponentials also give this workgroup's column sums of exp(K + u_t + v_{t-1});
// one exchange of those sums inside the batch element (exchange_columns); then
// every workgroup of the element forms v_t = log b + v_{t-1} - log colsum with
// the same bits.  Columns whose sum is below the floor take the exact
// max-shifted LSE (kernels.cu:629-671) through two more exchanges (column max,
// then sum); the decision is the same in every workgroup of the element
// because they all hold the same sums.  The batch-global stop test
// (torch_cuda.cpp:225-237) of iteration t-1 is evaluated during iteration t:
// wave 0 issues the loads of every workgroup's delta of t-1 before the row
// update and reads them after the exchange, so the test costs no wait of its
// own; when it fires, iteration t is discarded and (u_{t-1}, v_{t-1}) are the
// result.
constexpr int kDeltaPrefetch = 4;  // delta loads in flight per lane of wave 0 (covers 256 workgroups)

template <int VEC, int CH, int RPW, bool SCHED = false>
__global__ __launch_bounds__(kThreads) void forward(FwdResArgs a) {
    using R = Row<VEC, CH>;
    constexpr int PL = R::PL;
    constexpr int ROWS = kWaves * RPW;
    constexpr int GR = RPW < 4 ? RPW : 4;  // rows per reduction group
    // LDS: wave rows 8N | v 2N | log b N | column max N | u 2*ROWS | log a ROWS | scratch 32
    extern __shared__ float lds[];
    float* part = lds;
    float* lds_v = lds + kWaves * a.N;
    float* lds_lb = lds_v + 2 * a.N;
    float* lds_mx = lds_lb + a.N;
    float* lds_u = lds_mx + a.N;
    float* lds_la = lds_u + 2 * ROWS;
    float* scratch = lds_la + ROWS;  // [0] global delta, [1..kWaves] wave deltas, [16..] reductions
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int G = gridDim.x;
    const int gid = logical_group(a.W);
    const int b = gid / a.W;
    const int w = gid % a.W;
    const int row0 = w * a.R;
    const int rend = min(row0 + a.R, a.M);
    const size_t bM = size_t(b) * a.M;
    const size_t bN = size_t(b) * a.N;
    const bool check = a.tol > 0.0f;
    // Padding (columns >= N, rows >= rend) holds the value whose K is -inf.
    const float pad = a.kscale > 0.0f ? -INFINITY : INFINITY;
    announce_xcc(a.xchg, a.N, b, a.W, w, a.xcc_tag);

    float x[RPW][PL];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        const int i = row0 + wave + kWaves * k;
        if (i < rend) {
            R::load(a.X + (bM + i) * a.N, lane, a.N, x[k], 0.0f);
#pragma unroll
            for (int e = 0; e < PL; ++e)
                if (!R::valid(lane, e, a.N)) x[k][e] = pad;
        } else {
#pragma unroll
            for (int e = 0; e < PL; ++e) x[k][e] = pad;
        }
    }
    for (int l = threadIdx.x; l < ROWS; l += kThreads) {
        const int i = row0 + l;
        lds_la[l] = (i < rend && a.log_a) ? a.log_a[bM + i] : a.log_a_default;
        lds_u[l] = 0.0f;
        lds_u[ROWS + l] = 0.0f;
    }
    for (int j = threadIdx.x; j < a.N; j += kThreads) {
        lds_lb[j] = a.log_b ? a.log_b[bN + j] : a.log_b_default;
        lds_v[j] = 0.0f;
        lds_v[a.N + j] = 0.0f;
    }
    __syncthreads();
    float v[PL];
#pragma unroll
    for (int e = 0; e < PL; ++e) v[e] = 0.0f;
    // log a of the row this lane takes in each group of GR rows
    float lga_slot[RPW / GR];
#pragma unroll
    for (int g = 0; g < RPW / GR; ++g) lga_slot[g] = lds_la[wave + kWaves * (g * GR + slot_of_lane<GR>(lane))];
    float lse_slot[RPW / GR];  // the same row's log2-sum-exp of the last iteration (the next shift)
#pragma unroll
    for (int g = 0; g < RPW / GR; ++g) lse_slot[g] = 0.0f;
    float kscale2 = a.kscale * kLog2E;
    // scheduled runs: this iteration's scale, and the next one's already in flight
    float ks_it = a.kscale;
    float ks_next = (SCHED && a.max_iter > 0) ? a.kscale_t[0] : a.kscale;
    bool dead = false;
    const bool local =
        element_on_one_xcd(a.xchg, a.N, b, a.W, w, a.spin_limit, a.status, dead, scratch, a.xcc_tag, a.mark) &&
        a.local_ok;
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
        unsigned long long* ds = a.dxchg + size_t((t - 1) % kDeltaSlots) * G;
        unsigned long long dpre[kDeltaPrefetch];
        if (test && wave == 0) {
#pragma unroll
            for (int q = 0; q < kDeltaPrefetch; ++q) {
                const int g = lane + q * kWave;
                dpre[q] = g < G ? __hip_atomic_load(ds + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : tag_pack(0.0f, a.tag_base | unsigned(t - 1));
            }
        }
        // Row update (kernels.cu:503-545) and the shared-exponential column sums,
        // in base 2: y = K log2(e) + v log2(e), m = max_j y, s = sum_j 2^(y - m),
        // u = log a - ln2 (m + log2 s), and the column sums take 2^(y - m) a / s.
        // Rows go in groups of GR: their maxima and sums are reduced across the
        // wave together (transposed butterfly), and each lane then takes the
        // logarithm for one row of the group.
        float acc[PL], v2[PL];
#pragma unroll
        for (int e = 0; e < PL; ++e) {
            acc[e] = 0.0f;
            v2[e] = v[e] * kLog2E;
        }
        float uk[RPW];  // this wave's new u values; stored after the loop, which keeps it branch-free
#pragma unroll
        for (int g0 = 0; g0 < RPW; g0 += GR) {
            float y[GR][PL];
            // The shift m of a row's exponentials: its log2-sum-exp of the
            // previous iteration, which spares the row maximum and keeps the sum
            // near 1 once v settles; the row maximum itself in the first
            // iteration and whenever the shifted sum leaves [2^-30, 2^30] (a
            // large change of v or of the scale, a row without a finite score).
            // Within it the largest term is at least 2^-42, so every term that
            // matters is a normal float, and the sum is above the floor
            // (1e-12) that applies only to a maximum-shifted sum.
            auto row_max = [&](const float (&v2)[PL]) {
                float lm[GR];
#pragma unroll
                for (int r = 0; r < GR; ++r) {
                    lm[r] = -FLT_MAX;
#pragma unroll
                    for (int e = 0; e < PL; ++e) lm[r] = fmaxf(lm[r], fmaf(x[g0 + r][e], kscale2, v2[e]));
                }
                return transposed_reduce<GR>(lm, OpMax{});
            };
            auto shifted_exps = [&](float m, const float (&v2)[PL]) {
                float ls[GR];
#pragma unroll
                for (int r = 0; r < GR; ++r) {
                    const float mr = read_lane(m, lane_of_slot<GR>(r));
                    ls[r] = 0.0f;
#pragma unroll
                    for (int e = 0; e < PL; ++e) {
                        y[r][e] = __builtin_amdgcn_exp2f(fmaf(x[g0 + r][e], kscale2, v2[e]) - mr);
                        ls[r] += y[r][e];
                    }
                }
                return transposed_sum<GR>(ls);
            };
            const bool exact = t == 1 || !a.lagged_shift;
            float m_l = exact ? row_max(v2) : lse_slot[g0 / GR];
            float s_sum = shifted_exps(m_l, v2);
            if (!exact && !__all(s_sum >= 0x1p-30f && s_sum <= 0x1p30f)) {
                // v2 again, opaque to the compiler: kept from sharing the first
                // pass's products, whose registers the exponentials then reuse
                float v2r[PL];
#pragma unroll
                for (int e = 0; e < PL; ++e) {
                    v2r[e] = v2[e];
                    asm volatile("" : "+v"(v2r[e]));
                }
                m_l = row_max(v2r);
                s_sum = shifted_exps(m_l, v2r);
            }
            const float s_l = fmaxf(s_sum, sk::kSumFloor);
            const float lga_l = lga_slot[g0 / GR];
            const float lg2 = __builtin_amdgcn_logf(s_l);  // log2
            const float lse = m_l + lg2;
            lse_slot[g0 / GR] = lse;
            const float u_l = lga_l - kLn2 * lse;
            const float w_l = __builtin_amdgcn_exp2f(fmaf(lga_l, kLog2E, -lg2));  // a / s
#pragma unroll
            for (int r = 0; r < GR; ++r) {
                const float wr = read_lane(w_l, lane_of_slot<GR>(r));
                uk[g0 + r] = read_lane(u_l, lane_of_slot<GR>(r));
#pragma unroll
                for (int e = 0; e < PL; ++e) acc[e] = fmaf(y[r][e], wr, acc[e]);
            }
            // Materialise acc here: left alone, the compiler postpones the updates
            // to the end of the loop and keeps every group's exponentials live.
#pragma unroll
            for (int e = 0; e < PL; ++e) asm volatile("" : "+v"(acc[e]));
        }
        float dmax = 0.0f;
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            const int l = wave + kWaves * k;
            const int i = row0 + l;
            if (i < rend) {
                dmax = fmaxf(dmax, fabsf(uk[k] - lds_u[prev * ROWS + l]));
                if (lane == 0) {
                    lds_u[cur * ROWS + l] = uk[k];
                    if (a.u_hist) a.u_hist[(size_t(t - 1) * a.B + b) * a.M + i] = uk[k];
                }
            }
        }
        // The last readers of part (the previous exchange or exact fallback)
        // are behind the barrier that ends the previous iteration's exchange.
        R::store(part + wave * a.N, lane, a.N, acc);
        if (lane == 0) scratch[1 + wave] = dmax;
        __syncthreads();
        if (check && threadIdx.x == 0) {
            float d = scratch[1];
#pragma unroll
            for (int q = 1; q < kWaves; ++q) d = fmaxf(d, scratch[1 + q]);
            publish(a.dxchg + size_t(t % kDeltaSlots) * G + gid, d, a.tag_base | unsigned(t));
        }
        int low = 0;
        exchange_columns<kColRounds<PL>>(
            part, a.xchg + size_t(cur) * G * a.N, a.N, b, a.W, w, a.tag_base | unsigned(t), local, a.spin_limit,
            a.status, dead, a.mark,
            [&](int j, float cs) {
                if (cs >= sk::kColSumFloor && cs <= FLT_MAX) {
                    lds_v[cur * a.N + j] = lds_lb[j] + lds_v[prev * a.N + j] - logf(cs);
                } else {
                    lds_v[cur * a.N + j] = __builtin_nanf("");  // exact LSE below
                    low = 1;
                }
            });
        if (test && wave == 0) {
            float gmax = 0.0f;
#pragma unroll
            for (int q = 0; q < kDeltaPrefetch; ++q) {
                const int g = lane + q * kWave;
                if (g < G) {
                    float d = __uint_as_float(static_cast<unsigned>(dpre[q]));
                    if (static_cast<unsigned>(dpre[q] >> 32) != (a.tag_base | unsigned(t - 1)))
                        d = collect(ds + g, a.tag_base | unsigned(t - 1), a.spin_limit, a.status, dead, a.mark);
                    gmax = OpMaxNan{}(gmax, d);
                }
            }
            for (int g = lane + kDeltaPrefetch * kWave; g < G; g += kWave)
                gmax = OpMaxNan{}(gmax, collect(ds + g, a.tag_base | unsigned(t - 1), a.spin_limit, a.status,
                                                dead, a.mark));
            gmax = wave_reduce(gmax, OpMaxNan{});
            if (lane == 0) scratch[0] = gmax;
        }
        if (__syncthreads_or(low)) {
            // Exact column LSE of K + u_t over the element's rows: max, then sum.
            float cm[PL];
#pragma unroll
            for (int e = 0; e < PL; ++e) cm[e] = -FLT_MAX;
#pragma unroll
            for (int k = 0; k < RPW; ++k) {
                const int l = wave + kWaves * k;
                if (row0 + l >= rend) continue;
                const float u = lds_u[cur * ROWS + l];
#pragma unroll
                for (int e = 0; e < PL; ++e)
                    if (R::valid(lane, e, a.N)) cm[e] = fmaxf(cm[e], fmaf(x[k][e], ks_it, u));
            }
            tree_combine<VEC, CH>(cm, part, a.N, OpMax{});
            unsigned long long* fslot = a.fxchg + size_t(cur) * 2 * G * a.N;
            if (wave == 0) {
                unsigned long long* mine = fslot + size_t(gid) * a.N;
#pragma unroll
                for (int k = 0; k < CH; ++k)
#pragma unroll
                    for (int q = 0; q < VEC; ++q) {
                        const int col = R::col(lane, k) + q;
                        if (col < a.N) publish(mine + col, cm[k * VEC + q], a.tag_base | unsigned(t), local);
                    }
            }
            __syncthreads();
            for (int w2 = wave; w2 < a.W; w2 += kWaves) {
                float got[PL];
                collect_row<VEC, CH>(fslot + (size_t(b) * a.W + w2) * a.N, a.tag_base | unsigned(t), a.N,
                                     a.spin_limit, a.status, dead, got, a.mark);
                R::store(part + w2 * a.N, lane, a.N, got);
            }
            __syncthreads();
            for (int j = threadIdx.x; j < a.N; j += kThreads) {
                float mx = -FLT_MAX;
                for (int w2 = 0; w2 < a.W; ++w2) mx = fmaxf(mx, part[w2 * a.N + j]);
                lds_mx[j] = mx;
            }
            __syncthreads();
            float mxl[PL], sm[PL];
            R::load(lds_mx, lane, a.N, mxl, 0.0f);
#pragma unroll
            for (int e = 0; e < PL; ++e) sm[e] = 0.0f;
#pragma unroll
            for (int k = 0; k < RPW; ++k) {
                const int l = wave + kWaves * k;
                if (row0 + l >= rend) continue;
                const float u = lds_u[cur * ROWS + l];
#pragma unroll
                for (int e = 0; e < PL; ++e)
                    if (R::valid(lane, e, a.N)) sm[e] += safe_exp(fmaf(x[k][e], ks_it, u) - mxl[e]);
            }
            tree_combine<VEC, CH>(sm, part, a.N);
            unsigned long long* sslot = fslot + size_t(G) * a.N;
            if (wave == 0) {
                unsigned long long* mine = sslot + size_t(gid) * a.N;
#pragma unroll
                for (int k = 0; k < CH; ++k)
#pragma unroll
                    for (int q = 0; q < VEC; ++q) {
                        const int col = R::col(lane, k) + q;
                        if (col < a.N) publish(mine + col, sm[k * VEC + q], a.tag_base | unsigned(t), local);
                    }
            }
            __syncthreads();
            for (int w2 = wave; w2 < a.W; w2 += kWaves) {
                float got[PL];
                collect_row<VEC, CH>(sslot + (size_t(b) * a.W + w2) * a.N, a.tag_base | unsigned(t), a.N,
                                     a.spin_limit, a.status, dead, got, a.mark);
                R::store(part + w2 * a.N, lane, a.N, got);
            }
            __syncthreads();
            for (int j = threadIdx.x; j < a.N; j += kThreads) {
                const float vj = lds_v[cur * a.N + j];
                if (vj != vj) {
                    float s = 0.0f;
                    for (int w2 = 0; w2 < a.W; ++w2) s += part[w2 * a.N + j];
                    lds_v[cur * a.N + j] = lds_lb[j] - (lds_mx[j] + logf(fmaxf(s, sk::kSumFloor)));
                }
            }
            __syncthreads();
        }
        if (a.v_hist && w == 0)
            for (int j = threadIdx.x; j < a.N; j += kThreads)
                a.v_hist[(size_t(t - 1) * a.B + b) * a.N + j] = lds_v[cur * a.N + j];
        if (test && scratch[0] < a.tol) {  // the stop test of iteration t-1 fired
            used = t - 1;
            conv = 1;
            break;
        }
        R::load(lds_v + cur * a.N, lane, a.N, v, 0.0f);
    }
    if (check && conv == 0 && a.max_iter >= 1) {
        if (global_delta(a, a.max_iter, scratch, dead) < a.tol) conv = 1;  // the last iteration
    }

    // P = safe_exp(K + u + v) (kernels.cu:755-775) and this workgroup's share of
    // sum(P C), which workgroup 0 of the element adds up into the cost.
    const int par = used & 1;
    __syncthreads();
    const bool failed = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= a.mark;
    float vf[PL];
    R::load(lds_v + par * a.N, lane, a.N, vf, 0.0f);
    if (a.v_out && w == 0 && wave == 0) R::store(a.v_out + bN, lane, a.N, vf);
    const float csign = a.scores_kind < 0 ? 1.0f : -1.0f;  // C = -log_alpha
    float cacc = 0.0f;
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        const int l = wave + kWaves * k;
        const int i = row0 + l;
        if (i >= rend) continue;
        const float ui = lds_u[par * ROWS + l];
        if (a.u_out && lane == 0) a.u_out[bM + i] = ui;
        float pv[PL];
#pragma unroll
        for (int e = 0; e < PL; ++e) {
            const float lp = (x[k][e] * a.kscale + ui) + vf[e];
            pv[e] = a.return_log ? lp : safe_exp(lp);
            if (a.cost && R::valid(lane, e, a.N)) cacc = fmaf(pv[e], csign * x[k][e], cacc);
            if (failed) pv[e] = __builtin_nanf("");
        }
        if (a.plan) R::store(a.plan + (bM + i) * a.N, lane, a.N, pv);
    }
    if (a.cost) {
        const float cs = block_reduce<kWaves>(wave_sum(cacc), scratch + 16, OpSum{});
        if (threadIdx.x == 0) {
            const float s = element_sum(a.cwords, gid, w, a.W, failed ? __builtin_nanf("") : cs, a.result_tag,
                                        a.spin_limit, a.status, dead, a.mark);
            if (w == 0) a.cost[b] = s;
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *a.iters_used = failed ? -1 : used;  // -1: an exchange timed out, the outputs are NaN
        *a.converged = conv;
    }
}

}  // namespace res
}  // namespace dot_amd
