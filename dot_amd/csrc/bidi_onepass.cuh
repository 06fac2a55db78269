// One-pass bidirectional softmax: each input byte is read from HBM once.
//
// The two-sweep kernels (bidi_kernels.cuh) read sim twice in the forward and
// sim and grad_out twice in the backward (32 B per element per fwd+bwd against
// 20 for one pass).  Here a batch element is held in the registers of one
// group of kMembers = 32 workgroups while its column statistics are combined:
//
//   * groups: workgroup b belongs to group b % groups and is member b / groups.
//     The dispatcher places workgroup b on XCD b % 8, so with 8 groups every
//     group sits on one XCD (32 CUs, one 512-thread workgroup per CU) and its
//     exchange words stay in that XCD's L2; the kernels check the placement
//     (XCC ids announced at start) and fall back to agent-scope stores when
//     it does not hold.
//   * group g takes batch elements g, g + groups, ... in turn (a "stage" per
//     element).  Member m holds rows [32m, 32m + 32) of the element: wave w
//     rows 32m + 4w + j, j = 0..3, in the row-in-registers layout (row.cuh).
//   * column statistics: each wave folds its 4 rows per column, the 8 waves
//     are folded through LDS, every member publishes one word per column; the
//     owner of columns [32m, 32m + 32) (member m) combines the 32 members'
//     words in member order and publishes the result; every member collects
//     all results (reduce-scatter then all-gather, two tagged round trips).
//   * forward (fwd_kernel): the next element is loaded into a second register
//     buffer while the current one is exchanged and written; each row of the
//     current buffer is refilled with the element after next once written.
//   * backward (bwd_kernel): sim and grad_out of one element fill the
//     registers; phase A turns them into (t, c) with t = 2q - dot_r r and the
//     column-dot partials; phase B writes grad = (t - dot_c c) / tau and
//     refills each row with the next element's.
//
// Workgroups wait on other workgroups of their group, and the launch is a
// plain one (a cooperative launch costs ~18 us here).  When a wait passes its
// deadline (a member not yet resident because other work holds the CUs), the
// workgroup computes the element's column statistics itself by streaming the
// element's rows through the same per-member arithmetic in the same order
// (fallback_*), so the result is bitwise the one the exchange would have
// given; a late workgroup never turns into an error or a hang.
//
// Exchange words are 64-bit (value | tag << 32) with tag = epoch << 12 |
// (stage + 1) (stage 0: the XCC announce), so words of an earlier call never
// match; the caller hands in words cleared once plus a call epoch that grows
// per call on those words (dot_bidisoftmax_fwd_args.exchange).
//
// Semantics follow the two-sweep kernels (src/bidirectional_softmax/kernels.cu
// :90-242 forward, :249-411 backward): out = sqrt(1e-9 + r c) in the valid
// region [0, l1) x [0, l2), 0 elsewhere; statistics stored as planes (a
// reference point m and the sum of exp2(y2 - m)).
#pragma once

#include <cfloat>
#include <cstdint>

#include "bidi_kernels.cuh"
#include "resident.cuh"

#pragma clang fp contract(off)

namespace dot_amd {
namespace bidi {
namespace onepass {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;                  // 8
constexpr int kMembers = 32;                              // workgroups per group
constexpr int kRowsPerWave = 4;
constexpr int kRowsPerMember = kWaves * kRowsPerWave;     // 32
constexpr int kMaxRows = kMembers * kRowsPerMember;       // 1024
constexpr int kMaxCols = 1024;
constexpr int kOwn = kMaxCols / kMembers;                 // 32 columns owned per member
constexpr int kMaxGroups = 8;
constexpr int kStageBits = 12;
constexpr int kMaxStages = (1 << kStageBits) - 1;         // elements per group per call
constexpr unsigned kMaxEpoch = (1u << (32 - kStageBits)) - 1;
// Backward: waves [0, kPollWaves) wait on the exchange while the others load
// every wave's rows of the next grad_out into LDS (their loads then do not
// queue ahead of the polls: a wave's vector loads complete in issue order).
constexpr int kPollWaves = kWaves / 2;
constexpr int kPreRows = kRowsPerWave;
// Forward: rows of each wave's element after next loaded into LDS while the
// exchange runs.
constexpr int kFwdPreRows = 2;

// Exchange words: partials [groups][2][kMembers][kMaxCols], results
// [groups][2][kMaxCols], XCC announces [groups][kMembers]; the middle 2 is the
// stage parity.
constexpr size_t kPartWords = size_t(kMaxGroups) * 2 * kMembers * kMaxCols;
constexpr size_t kResWords = size_t(kMaxGroups) * 2 * kMaxCols;
constexpr size_t kXccWords = size_t(kMaxGroups) * kMembers;
constexpr size_t kExchangeWords = kPartWords + kResWords + kXccWords;

struct Exchange {
    unsigned long long* words;  // kExchangeWords
    int groups;
    unsigned epoch;             // 1 .. kMaxEpoch
    int wait_ticks;             // deadline of a wait in s_memrealtime ticks (10 ns); < 0: never wait
    int local_ok;               // XCD-local exchange stores allowed (local_exchange_allowed)
};

__device__ __forceinline__ unsigned long long* part_row(const Exchange& x, int g, int p, int m) {
    return x.words + ((size_t(g) * 2 + p) * kMembers + m) * kMaxCols;
}
__device__ __forceinline__ unsigned long long* res_row(const Exchange& x, int g, int p) {
    return x.words + kPartWords + (size_t(g) * 2 + p) * kMaxCols;
}
__device__ __forceinline__ unsigned long long* xcc_word(const Exchange& x, int g, int m) {
    return x.words + kPartWords + kResWords + size_t(g) * kMembers + m;
}

__device__ __forceinline__ long long now_ticks() { return (long long)__builtin_amdgcn_s_memrealtime(); }

// Waits until both words carry `tag`; false once `deadline` has passed (or at
// once when wait_ticks < 0).
__device__ __forceinline__ bool poll2(unsigned long long* p0, unsigned long long* p1, unsigned tag,
                                      long long deadline, bool never, float& v0, float& v1) {
    if (never) return false;
    for (;;) {
        const unsigned long long x0 = __hip_atomic_load(p0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long x1 = __hip_atomic_load(p1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (unsigned(x0 >> 32) == tag && unsigned(x1 >> 32) == tag) {
            v0 = __uint_as_float(unsigned(x0));
            v1 = __uint_as_float(unsigned(x1));
            return true;
        }
        if (now_ticks() > deadline) return false;
        // rounds back to back: each is a memory round trip already
    }
}

// Waits until all four words carry `tag` (see poll2).
__device__ __forceinline__ bool poll4(unsigned long long* const (&w)[4], unsigned tag, long long deadline, bool never,
                                      float (&v)[4]) {
    if (never) return false;
    for (;;) {
        unsigned long long x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = __hip_atomic_load(w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool all = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) all = all && unsigned(x[i] >> 32) == tag;
        if (all) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(unsigned(x[i]));
            return true;
        }
        if (now_ticks() > deadline) return false;
    }
}

// Workgroup barrier for data passed through LDS only: this wave's LDS
// accesses complete (lgkmcnt 0), then s_barrier, with compiler barriers on
// both sides.  Unlike __syncthreads() (a workgroup release fence) it does not
// wait for the wave's outstanding vector-memory loads into LDS, so a wave may
// pass it while its prefetch is still in flight; the prefetched words are read
// only after a later vmcnt wait and barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt at their maxima (no wait)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The OR over the workgroup's waves of a wave-uniform `bits` (every lane of
// wave `wave` writes the same vote), in every thread; one barrier.
__device__ __forceinline__ int block_or(int bits, int* votes, int wave) {
    votes[wave] = bits;
    lds_barrier();
    const int4 v0 = reinterpret_cast<const int4*>(votes)[0];
    const int4 v1 = reinterpret_cast<const int4*>(votes)[1];
    return v0.x | v0.y | v0.z | v0.w | v1.x | v1.y | v1.z | v1.w;
}

// Wave-uniform reads of inputs that no kernel of this file writes (lengths,
// the backward's statistics) through the scalar unit: a vector load would wait
// behind every row load the wave has in flight (vector loads complete in
// order), stalling a stage until the next element's rows have arrived.
__device__ __forceinline__ float scalar_load(const float* p) {
    return *(const __attribute__((address_space(4))) float*)(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ void scalar_extent(const int32_t* lengths, int b, int L1, int L2, int& l1, int& l2) {
    if (!lengths) {  // no lengths: every element is full
        l1 = L1;
        l2 = L2;
        return;
    }
    const auto* q = (const __attribute__((address_space(4))) int32_t*)(reinterpret_cast<uintptr_t>(lengths + 2 * b));
    l1 = min(max(q[0], 0), L1);
    l2 = min(max(q[1], 0), L2);
}

// Valid rows and columns of element b; a full tile (no lengths) has constant
// ones.
__device__ __forceinline__ void extent(const int32_t* lengths, int b, int L1, int L2, bool full_tile, int& l1,
                                       int& l2) {
    if (full_tile) {
        l1 = L1;
        l2 = L2;
    } else {
        scalar_extent(lengths, b, L1, L2, l1, l2);
    }
}

// Online (max, sum) state of base-2 exponentials, one exponential per update:
// after a sequence of updates s * 2^m is the sum of 2^y.  Starting state
// (-FLT_MAX, 0); y = -inf adds nothing.
__device__ __forceinline__ void online_add(float& m, float& s, float y) {
    const float d = y - m;
    const float x = __builtin_amdgcn_exp2f(-fabsf(d));
    const bool gt = d > 0.0f;
    s = gt ? fmaf(s, x, 1.0f) : s + x;
    m = gt ? y : m;
}

// log2 of the sum of a (m, s) state; -inf when empty.
__device__ __forceinline__ float state_lse(float m, float s) {
    return s > 0.0f ? m + __builtin_amdgcn_logf(s) : -INFINITY;
}

// Rows of one batch element through a buffer resource: 32-bit offsets inside
// the element (one VGPR of lane offset, no 64-bit addresses per row), and a
// load past the element's end reads 0 instead of faulting, so the lanes past
// L2 on its last row need no clamp.
typedef unsigned v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t element_rsrc(const float* base, size_t elem, int e) {
    // the address is wave-uniform; readfirstlane lets the compiler keep the
    // descriptor in scalar registers (no per-lane loop around each access)
    const uintptr_t p = reinterpret_cast<uintptr_t>(base + size_t(e) * elem);
    const unsigned lo = __builtin_amdgcn_readfirstlane(unsigned(p));
    const unsigned hi = __builtin_amdgcn_readfirstlane(unsigned(p >> 32));
    float* u = reinterpret_cast<float*>((uintptr_t(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, 0, __builtin_amdgcn_readfirstlane(unsigned(elem * 4)), 0x00020000);
}

// Row `row` (< L1) of the element: lane l gets columns kk*256 + 4l .. +3; the
// lanes past L2 get whatever follows (the caller masks them).
// A value the compiler cannot see through, so that the per-row offsets are
// formed where they are used instead of being hoisted out of the element loop
// and held (or spilled) for all rows at once.
__device__ __forceinline__ unsigned fresh(unsigned x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ int fresh(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

// The lane's index in its wave, computed (two VALU instructions) at each use:
// inside the element loops thread indices are formed from it and the
// wave-uniform wave index, so that no per-lane index is held across the loop
// (a held one is spilled, and its reload is a memory load that completes only
// after every row load the wave has in flight).
__device__ __forceinline__ int lane_now() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

template <int CH>
__device__ __forceinline__ void load_row(__amdgpu_buffer_rsrc_t r, int row, int L2, int lane, float (&x)[4 * CH]) {
    const unsigned off = fresh(unsigned(row) * unsigned(L2) * 4u + unsigned(lane) * 16u);
#pragma unroll
    for (int kk = 0; kk < CH; ++kk) {
        const v4u t = __builtin_amdgcn_raw_buffer_load_b128(r, off + kk * 1024u, 0, 0);
        x[4 * kk + 0] = __uint_as_float(t.x);
        x[4 * kk + 1] = __uint_as_float(t.y);
        x[4 * kk + 2] = __uint_as_float(t.z);
        x[4 * kk + 3] = __uint_as_float(t.w);
    }
}

// The words of element_rsrc's descriptor (base, stride 0, byte size, the
// same flags), wave-uniform, for the LDS loads below.
__device__ __forceinline__ v4u element_words(const float* base, size_t elem, int e) {
    const uintptr_t p = reinterpret_cast<uintptr_t>(base + size_t(e) * elem);
    v4u w;
    w.x = __builtin_amdgcn_readfirstlane(unsigned(p));
    w.y = __builtin_amdgcn_readfirstlane(unsigned(p >> 32)) & 0xffffu;
    w.z = __builtin_amdgcn_readfirstlane(unsigned(elem * 4));
    w.w = 0x00020000u;
    return w;
}

// load_row into LDS instead of registers: 16-byte buffer loads that write LDS
// directly (M0 = the wave-uniform LDS byte address; lane l's 16 bytes land at
// M0 + 16 l, so columns kk*256 + 4l .. +3 sit at float offset kk*256 + 4l of
// `dst`, the layout load_row gives the registers; no instruction offset, which
// would move the LDS address too).  Issued from inline
// assembly so that the compiler adds no wait for them: the data is there once
// this wave has waited for vmcnt(0), and other waves may read it after a
// barrier that follows that wait.  M0 is restored after each load.
template <int CH>
__device__ __forceinline__ void load_row_lds(v4u r, int row, int L2, int lane, unsigned dst) {
    const unsigned off = fresh(unsigned(row) * unsigned(L2) * 4u + unsigned(lane) * 16u);
#pragma unroll
    for (int kk = 0; kk < CH; ++kk) {
        unsigned saved;
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(dst + kk * 1024u), "v"(off + kk * 1024u), "s"(r)
            : "memory");
    }
}

// Non-temporal store of a row's columns < L2 (L2 % 4 == 0).
template <int CH>
__device__ __forceinline__ void store_row(__amdgpu_buffer_rsrc_t r, int row, int L2, int lane,
                                          const float (&x)[4 * CH]) {
    const unsigned off = fresh(unsigned(row) * unsigned(L2) * 4u + unsigned(lane) * 16u);
#pragma unroll
    for (int kk = 0; kk < CH; ++kk) {
        const v4u t = {__float_as_uint(x[4 * kk + 0]), __float_as_uint(x[4 * kk + 1]), __float_as_uint(x[4 * kk + 2]),
                       __float_as_uint(x[4 * kk + 3])};
        if (kk * 256 + 4 * lane < L2) __builtin_amdgcn_raw_buffer_store_b128(t, r, off + kk * 1024u, 0, 2);
    }
}

// Fold of the 8 waves' (m, s) column states in LDS (lm, ls: [kWaves][kMaxCols])
// for columns 2t and 2t + 1: the maximum over the waves, then the rescaled
// sums in wave order; columns >= L2 are empty.
__device__ __forceinline__ void fold_lse(const float* lm, const float* ls, int t, int L2, float& l0, float& l1) {
    if (2 * t >= L2) {
        l0 = l1 = -INFINITY;
        return;
    }
    const float2* pm = reinterpret_cast<const float2*>(lm);
    const float2* ps = reinterpret_cast<const float2*>(ls);
    float2 mw[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mw[w] = pm[w * (kMaxCols / 2) + t];
    float M0 = mw[0].x, M1 = mw[0].y;
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        M0 = fmaxf(M0, mw[w].x);
        M1 = fmaxf(M1, mw[w].y);
    }
    float S0 = 0.0f, S1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const float2 sw = ps[w * (kMaxCols / 2) + t];
        S0 += sw.x * __builtin_amdgcn_exp2f(mw[w].x - M0);
        S1 += sw.y * __builtin_amdgcn_exp2f(mw[w].y - M1);
    }
    l0 = state_lse(M0, S0);
    l1 = state_lse(M1, S1);
}

struct FwdArgs1 {
    const float* sim;
    const int32_t* lengths;
    float sc;  // log2(e) / tau
    int B, L1, L2;
    float* out;
    float* row_stats;  // [B,2,L1]
    float* col_stats;  // [B,2,L2]
    Exchange x;
};

// Per-wave column state of a wave's rows (scaled and masked): the column
// maximum over the rows (from -FLT_MAX, in row order), then the sum of
// exp2(y - max) in row order.  The exchange path applies column_max and
// column_sum to rows held in registers, the fallback to rows streamed twice;
// the arithmetic and its order are the same, so their results agree bitwise.
template <int PL>
__device__ __forceinline__ void column_max(float (&cm)[PL], const float (&y)[PL]) {
#pragma unroll
    for (int q = 0; q < PL; ++q) cm[q] = fmaxf(cm[q], y[q]);
}
template <int PL>
__device__ __forceinline__ void column_sum(float (&cs)[PL], const float (&cm)[PL], const float (&y)[PL]) {
#pragma unroll
    for (int q = 0; q < PL; ++q) cs[q] += __builtin_amdgcn_exp2f(y[q] - cm[q]);
}

// y2 = sim * sc for this lane's columns of row i, -inf outside the valid
// region (row >= l1 or column >= l2).  `full` (a valid row whose every lane
// column is valid, wave-uniform) skips the masks.
template <class R>
__device__ __forceinline__ void scale_mask(float (&v)[R::PL], float sc, bool row_ok, int lane, int l2, bool full) {
    if (full) {
#pragma unroll
        for (int q = 0; q < R::PL; ++q) v[q] *= sc;
    } else {
#pragma unroll
        for (int q = 0; q < R::PL; ++q) v[q] = (row_ok && R::valid(lane, q, l2)) ? v[q] * sc : -INFINITY;
    }
}

// Forward column statistics of element e computed by this workgroup alone
// (a wait passed its deadline): the per-member states of all 32 members,
// merged in member order exactly as the owners merge the published words.
// Leaves log2-sum-exp2 of each column in clse; when `own` is set, also does
// the owner's part for this member's columns (publish the results, store the
// column statistics).  Contains barriers.
template <int CH, bool FW>
__device__ void fwd_fallback(const FwdArgs1& a, int e, int l1, int l2, int g, int m, int p, unsigned tag, bool local,
                             bool own, float* lm, float* ls, float* clse, int wave) {
    using R = Row<4, CH>;
    // FW (full tile): no lengths, 1024 rows of 256 * CH columns; the extents
    // are then constants and every row and column check folds away
    const int L2 = FW ? 4 * kWave * CH : a.L2;
    const int L1 = FW ? kMaxRows : a.L1;
    const int lane = lane_now();
    const int t = wave * kWave + lane;
    const auto rs = element_rsrc(a.sim, size_t(L1) * L2, e);
    float M0 = -FLT_MAX, S0 = 0.0f, M1 = -FLT_MAX, S1 = 0.0f;
    for (int mm = 0; mm < kMembers; ++mm) {
        float cm[R::PL], cs[R::PL];
#pragma unroll
        for (int q = 0; q < R::PL; ++q) {
            cm[q] = -FLT_MAX;
            cs[q] = 0.0f;
        }
        const bool full_cols = l2 == 4 * kWave * CH;
        // one row in registers at a time (the caller's buffers stay live)
#pragma unroll 1
        for (int pass = 0; pass < 2; ++pass) {
#pragma unroll 1
            for (int j = 0; j < kRowsPerWave; ++j) {
                const int i = mm * kRowsPerMember + wave * kRowsPerWave + j;
                float v[R::PL];
                load_row<CH>(rs, min(i, L1 - 1), L2, lane, v);
                scale_mask<R>(v, a.sc, i < l1, lane, l2, full_cols && i < l1);
                if (pass == 0)
                    column_max(cm, v);
                else
                    column_sum(cs, cm, v);
            }
        }
        __syncthreads();  // the previous member's fold has been read
        R::store(lm + wave * kMaxCols, lane, L2, cm);
        R::store(ls + wave * kMaxCols, lane, L2, cs);
        __syncthreads();
        float l0, l1v;
        fold_lse(lm, ls, t, L2, l0, l1v);
        online_add(M0, S0, l0);
        online_add(M1, S1, l1v);
    }
    const float L0 = state_lse(M0, S0), L1v = state_lse(M1, S1);
    clse[2 * t] = L0;
    clse[2 * t + 1] = L1v;
    if (own && 2 * t >= kOwn * m && 2 * t < kOwn * (m + 1)) {
        unsigned long long* r = res_row(a.x, g, p);
        res::publish(r + 2 * t, L0, tag, local);
        res::publish(r + 2 * t + 1, L1v, tag, local);
        if (2 * t < L2) {
            float* cst = a.col_stats + size_t(e) * 2 * L2;
            cst[2 * t] = M0;
            cst[2 * t + 1] = M1;
            cst[L2 + 2 * t] = S0;
            cst[L2 + 2 * t + 1] = S1;
        }
    }
    __syncthreads();
}

// Deadline of the XCD check (s_memrealtime ticks of 10 ns): the members of a
// launch start within a few microseconds of each other.
constexpr int kXcdCheckTicks = 500;

// Run by one wave at the start of a launch, before it issues any row load
// (its poll then queues behind nothing): *flag = 1 when every member of group
// g runs on this workgroup's XCD (their announced XCC ids), else 0; a member
// not yet announced by the deadline reads as "no" and leaves the call's
// exchange at agent scope.  The other waves read the flag after a barrier.
// Each member decides alone: one that sees all 32 ids on its own XCD knows
// that every reader of its words is there, and a member that does not uses
// agent-scope stores, which every reader sees.
__device__ __forceinline__ void check_group_xcd(const Exchange& x, int g, unsigned tag0, bool never, int* flag) {
    const int me = res::xcc_id();
    const long long deadline = now_ticks() + kXcdCheckTicks;
    const int lane = lane_now();
    int same = 1;
    if (lane < kMembers) {
        float v0, v1;
        unsigned long long* w = xcc_word(x, g, lane);
        same = poll2(w, w, tag0, deadline, never, v0, v1) && __float_as_int(v0) == me;
    }
    *flag = __all(same);  // every lane: the same value
}

template <int CH, bool FW>
__global__ __launch_bounds__(kThreads, 1) void fwd_kernel(FwdArgs1 a) {
    using R = Row<4, CH>;
    // FW (full tile): no lengths, 1024 rows of 256 * CH columns; the extents
    // are then constants and every row and column check folds away
    const int L2 = FW ? 4 * kWave * CH : a.L2;
    const int L1 = FW ? kMaxRows : a.L1;
    constexpr int PL = R::PL;
    __shared__ __align__(16) float lm[kWaves * kMaxCols];
    __shared__ __align__(16) float ls[kWaves * kMaxCols];
    // rows 0 .. kFwdPreRows - 1 of each wave's element after next, loaded
    // during the exchange
    __shared__ __align__(16) float pre[kWaves * kFwdPreRows * kMaxCols];
    __shared__ float rsv[kMembers][kOwn + 1];
    __shared__ __align__(16) float clse[kMaxCols];
    __shared__ int flag;
    __shared__ __align__(16) int votes[kWaves];
    __shared__ int rsflag[kPollWaves];  // (element + 1) << 1 | failed, per polling wave
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int t = threadIdx.x;
    const int G = a.x.groups;
    const int g = blockIdx.x % G;
    const int m = blockIdx.x / G;
    const int n = (a.B - g + G - 1) / G;  // this group's elements
    const unsigned pre0 = unsigned(uintptr_t((__attribute__((address_space(3))) float*)(pre)));
    if (n <= 0) return;
    const bool never = a.x.wait_ticks < 0;
    const unsigned tag0 = a.x.epoch << kStageBits;
    if (t == 0) res::publish(xcc_word(a.x, g, m), __int_as_float(res::xcc_id()), tag0);
    const int row0 = m * kRowsPerMember + wave * kRowsPerWave;
    float X[kRowsPerWave][PL], Y[kRowsPerWave][PL];
    // rows of element k of this group (past the last element: row 0 of element
    // `kc`, a cache hit, so that every load is unconditional)
    const size_t elem = size_t(L1) * L2;
    auto load = [&](int k, int kc, float(&buf)[kRowsPerWave][PL]) {
        const bool real = k < n;
        const auto rs = element_rsrc(a.sim, elem, g + G * (real ? k : kc));
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) load_row<CH>(rs, real ? min(row0 + j, L1 - 1) : 0, L2, lane, buf[j]);
    };
    if (wave == kWaves - 1) check_group_xcd(a.x, g, tag0, never, &flag);
    if (t < kPollWaves) rsflag[t] = 0;  // read after the first element's barriers
    load(0, 0, X);
    load(1, 0, Y);
    bool local = false;  // set at element 0's first barrier from the check's flag

    auto stage = [&](int k, float(&buf)[kRowsPerWave][PL]) {
        // thread indices re-formed per element: addresses derived from them are
        // computed here, not hoisted out of the element loop and spilled
        const int lane = lane_now();
        const int t = wave * kWave + lane;
        const int e = g + G * k;
        const unsigned tag = tag0 | unsigned(k + 1);
        const int p = k & 1;
        int l1, l2;
        extent(a.lengths, e, L1, L2, FW, l1, l2);
        // ---- row statistics and this wave's column states
        float rl[kRowsPerWave];
        float cm[PL], cs[PL];
#pragma unroll
        for (int q = 0; q < PL; ++q) {
            cm[q] = -FLT_MAX;
            cs[q] = 0.0f;
        }
        float* rst = a.row_stats + size_t(e) * 2 * L1;
        const bool full_cols = l2 == 4 * kWave * CH;
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) {
            const int i = row0 + j;
            scale_mask<R>(buf[j], a.sc, i < l1, lane, l2, full_cols && i < l1);
            column_max(cm, buf[j]);
        }
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) column_sum(cs, cm, buf[j]);
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) {
            const int i = row0 + j;
            float ml = -FLT_MAX;
#pragma unroll
            for (int q = 0; q < PL; ++q) ml = fmaxf(ml, buf[j][q]);
            const float rm = wave_max(ml);
            float sl = 0.0f;
#pragma unroll
            for (int q = 0; q < PL; ++q) sl += __builtin_amdgcn_exp2f(buf[j][q] - rm);
            const float rs = wave_sum(sl);
            rl[j] = rm + __builtin_amdgcn_logf(rs);
            if (i < l1) {  // wave-uniform
                rst[i] = rm;
                rst[L1 + i] = rs;
            }
        }
        // ---- fold the waves, publish this member's column words
        R::store(lm + wave * kMaxCols, lane, L2, cm);
        R::store(ls + wave * kMaxCols, lane, L2, cs);
        __syncthreads();
        if (k == 0) local = flag != 0 && a.x.local_ok;
        {
            float l0, l1v;
            fold_lse(lm, ls, t, L2, l0, l1v);
            unsigned long long* dst = part_row(a.x, g, p, m) + 2 * t;
            res::publish(dst, l0, tag, local);
            res::publish(dst + 1, l1v, tag, local);
        }
        const long long deadline = now_ticks() + a.x.wait_ticks;
        // ---- the first rows of every wave's element after next, into LDS
        // by the non-polling waves: HBM traffic while the exchange runs, not
        // queued ahead of any poll
        const int kn = k + 2;
        const bool real = kn < n;
        if (wave >= kPollWaves && real) {
            const v4u rw = element_words(a.sim, elem, g + G * kn);
            constexpr int per = kWaves / (kWaves - kPollWaves);
#pragma unroll
            for (int q = 0; q < per; ++q) {
                const int tw = (wave - kPollWaves) * per + q;
#pragma unroll
                for (int j = 0; j < kFwdPreRows; ++j)
                    load_row_lds<CH>(rw, min(m * kRowsPerMember + tw * kRowsPerWave + j, L1 - 1), L2, lane,
                                     pre0 + unsigned(tw * kFwdPreRows + j) * kMaxCols * 4u);
            }
        }
        // ---- reduce-scatter (waves < kPollWaves): member m owns columns
        // [32m, 32m + 32); thread t < 256 reads members 4h .. 4h + 3 (h = t / 32);
        // then the owner's merge and the all-gather.  The polling waves meet
        // through LDS flags, not a workgroup barrier: the other waves are
        // still issuing their loads.
        int fails = 0;  // bit 1: a reduce-scatter wait expired; bit 0: an all-gather wait
        if (wave < kPollWaves) {
            const int c = t & (kOwn - 1);
            const int h = t >> 5;
            unsigned long long* const w[4] = {
                part_row(a.x, g, p, 4 * h) + kOwn * m + c, part_row(a.x, g, p, 4 * h + 1) + kOwn * m + c,
                part_row(a.x, g, p, 4 * h + 2) + kOwn * m + c, part_row(a.x, g, p, 4 * h + 3) + kOwn * m + c};
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const bool ok = poll4(w, tag, deadline, never, v);
#pragma unroll
            for (int i = 0; i < 4; ++i) rsv[4 * h + i][c] = v[i];
            const int mine = ((k + 1) << 1) | (__ballot(!ok) != 0 ? 1 : 0);
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's rsv values are written
            __hip_atomic_store(&rsflag[wave], mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll 1
            for (int q = 0; q < kPollWaves; ++q) {
                int f;
                do {
                    f = __hip_atomic_load(&rsflag[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                } while ((f >> 1) != k + 1);
                fails |= (f & 1) << 1;
            }
            asm volatile("" ::: "memory");  // rsv is read after the flags
            if (!fails) {
                if (t < kOwn) {
                    float M = -FLT_MAX, S = 0.0f;
#pragma unroll 8
                    for (int q = 0; q < kMembers; ++q) online_add(M, S, rsv[q][t]);
                    const int col = kOwn * m + t;
                    res::publish(res_row(a.x, g, p) + col, state_lse(M, S), tag, local);
                    if (col < L2) {
                        float* cst = a.col_stats + size_t(e) * 2 * L2;
                        cst[col] = M;
                        cst[L2 + col] = S;
                    }
                }
                // ---- all-gather: thread t < 256 reads columns 4t .. 4t + 3
                unsigned long long* r = res_row(a.x, g, p) + 4 * t;
                unsigned long long* const wr[4] = {r, r + 1, r + 2, r + 3};
                float u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                const bool ok2 = poll4(wr, tag, deadline, never, u);
                *reinterpret_cast<float4*>(clse + 4 * t) = make_float4(u[0], u[1], u[2], u[3]);
                fails |= __ballot(!ok2) != 0 ? 1 : 0;
            }
        }
        fails = block_or(fails, votes, wave);
        if (fails) fwd_fallback<CH, FW>(a, e, l1, l2, g, m, p, tag, local, (fails & 2) != 0, lm, ls, clse, wave);
        // ---- write; each row is refilled with the element after next (its
        // first rows from LDS, once the loading waves have waited for them and
        // passed a barrier)
        if (wave >= kPollWaves && real) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        lds_barrier();
        const auto rs = element_rsrc(a.sim, elem, g + G * (real ? kn : k));
        const auto ro = element_rsrc(a.out, elem, e);
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) {
            const int i = row0 + j;
            float o[PL];
            const int z = fresh(0);  // column values read per row (see row_q)
            const bool full = full_cols && i < l1;
#pragma unroll
            for (int kk = 0; kk < CH; ++kk) {
                float cl[4];
                R::chunk(clse + z, lane, kk, L2, cl);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int ee = 4 * kk + q;
                    const float y = buf[j][ee];
                    const float x = (y - rl[j]) + (y - cl[q]);
                    o[ee] = __builtin_amdgcn_sqrtf(fmaf(__builtin_amdgcn_exp2f(x), 1.0f, kEps));
                }
            }
            if (!full) {
#pragma unroll
                for (int ee = 0; ee < PL; ++ee) o[ee] = (i < l1 && R::valid(lane, ee, l2)) ? o[ee] : 0.0f;
            }
            if (i < L1) store_row<CH>(ro, i, L2, lane, o);
            if (j < kFwdPreRows && real) {
                const float* src = pre + (wave * kFwdPreRows + j) * kMaxCols + 4 * lane;
#pragma unroll
                for (int kk = 0; kk < CH; ++kk) {
                    const float4 v = *reinterpret_cast<const float4*>(src + kk * 256);
                    buf[j][4 * kk + 0] = v.x;
                    buf[j][4 * kk + 1] = v.y;
                    buf[j][4 * kk + 2] = v.z;
                    buf[j][4 * kk + 3] = v.w;
                }
            } else {
                load_row<CH>(rs, real ? min(i, L1 - 1) : 0, L2, lane, buf[j]);
            }
        }
    };
    for (int k = 0; k < n; k += 2) {
        stage(k, X);
        if (k + 1 < n) stage(k + 1, Y);
    }
}

struct BwdArgs1 {
    const float* sim;
    const float* grad_out;
    const int32_t* lengths;
    float sc, inv_T;
    int B, L1, L2;
    const float* row_stats;  // [B,2,L1] as the forward wrote them
    const float* col_stats;  // [B,2,L2]
    float* grad_sim;
    Exchange x;
};

// log2 of a softmax denominator from its stored (reference point, sum) pair:
// r = exp2(y2 - log_norm); +inf (r = 0) for an empty row or column.
__device__ __forceinline__ float log_norm(float m, float s) {
    return s > 0.0f ? m + __builtin_amdgcn_logf(s) : INFINITY;
}

// row_q for a row with no masked entry (the same arithmetic, no selects).
template <int CH>
__device__ __forceinline__ void row_q_full(float (&y)[4 * CH], float (&gr)[4 * CH], float (&r)[4 * CH], float rl,
                                           int lane, int L2, float sc, const float* lcl) {
    using R = Row<4, CH>;
    const int z = fresh(0);
#pragma unroll
    for (int kk = 0; kk < CH; ++kk) {
        float cl[4];
        R::chunk(lcl + z, lane, kk, L2, cl);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int e = 4 * kk + qq;
            const float y2 = y[e] * sc;
            const float rr = __builtin_amdgcn_exp2f(y2 - rl);
            const float cc = __builtin_amdgcn_exp2f(y2 - cl[qq]);
            const float o = __builtin_amdgcn_sqrtf(fmaf(rr, cc, kEps));
            const float d = (gr[e] * 0.5f) * __builtin_amdgcn_rcpf(o);
            gr[e] = (d * rr) * cc;
            r[e] = rr;
            y[e] = cc;
        }
    }
}

// q = d r c (with d = g / (2 out), kernels.cu:249-274) for one row, in place:
// y (sim) becomes c and gr (grad_out) becomes q; r is written out.  r and c
// are 0 outside the valid region.  Both the exchange path and the fallback run
// this, so their column dots agree bitwise.
template <int CH>
__device__ __forceinline__ void row_q(float (&y)[4 * CH], float (&gr)[4 * CH], float (&r)[4 * CH], float rl,
                                      bool row_ok, int lane, int l2, int L2, float sc, const float* lcl, bool full) {
    if (full) {  // a valid row whose every lane column is valid: no masks
        row_q_full<CH>(y, gr, r, rl, lane, L2, sc, lcl);
        return;
    }
    using R = Row<4, CH>;
    // read per row: the same values for every row, which the compiler would
    // otherwise load once and hold in registers for all rows
    const int z = fresh(0);
#pragma unroll
    for (int kk = 0; kk < CH; ++kk) {
        float cl[4];
        R::chunk(lcl + z, lane, kk, L2, cl);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int e = 4 * kk + qq;
            const bool ok = row_ok && R::valid(lane, e, l2);
            const float y2 = y[e] * sc;
            const float rr = ok ? __builtin_amdgcn_exp2f(y2 - rl) : 0.0f;
            const float cc = ok ? __builtin_amdgcn_exp2f(y2 - cl[qq]) : 0.0f;
            const float o = __builtin_amdgcn_sqrtf(fmaf(rr, cc, kEps));
            const float d = ok ? (gr[e] * 0.5f) * __builtin_amdgcn_rcpf(o) : 0.0f;
            gr[e] = (d * rr) * cc;
            r[e] = rr;
            y[e] = cc;
        }
    }
}

// Adds a row's q to this wave's column partials in LDS (`dst`, the wave's
// kMaxCols floats): the partials live there instead of in 16 registers per
// lane.  Row 0 of a member starts the sum (0 + q, as a register sum would).
template <int CH>
__device__ __forceinline__ void acc_row(float* dst, int lane, int L2, const float (&q)[4 * CH], bool first) {
#pragma unroll
    for (int kk = 0; kk < CH; ++kk) {
        const int c = kk * 256 + 4 * lane;
        if (c < L2) {
            float4 v = first ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : *reinterpret_cast<const float4*>(dst + c);
            v.x += q[4 * kk + 0];
            v.y += q[4 * kk + 1];
            v.z += q[4 * kk + 2];
            v.w += q[4 * kk + 3];
            *reinterpret_cast<float4*>(dst + c) = v;
        }
    }
}

// Column dots of element e by this workgroup alone (see fwd_fallback): leaves
// them in ldc, and with `own` publishes this member's results.  Contains
// barriers.
template <int CH, bool FW>
__device__ void bwd_fallback(const BwdArgs1& a, int e, int l1, int l2, int g, int m, int p, unsigned tag,
                             bool local, bool own, float* lacc, const float* lcl, float* ldc, int wave) {
    using R = Row<4, CH>;
    const int L2 = FW ? 4 * kWave * CH : a.L2;  // full-width rows: a constant
    constexpr int PL = R::PL;
    const int lane = lane_now();
    const int t = wave * kWave + lane;
    const float* rst = a.row_stats + size_t(e) * 2 * a.L1;
    const auto ry = element_rsrc(a.sim, size_t(a.L1) * L2, e);
    const auto rg = element_rsrc(a.grad_out, size_t(a.L1) * L2, e);
    float s0 = 0.0f, s1 = 0.0f;
    for (int mm = 0; mm < kMembers; ++mm) {
        __syncthreads();  // the previous member's partials have been read
        // one row in registers at a time (the caller's buffers stay live)
#pragma unroll 1
        for (int j = 0; j < kRowsPerWave; ++j) {
            const int i = mm * kRowsPerMember + wave * kRowsPerWave + j;
            const bool row_ok = i < l1;
            float y[PL], gr[PL], r[PL];
            load_row<CH>(ry, min(i, a.L1 - 1), L2, lane, y);
            load_row<CH>(rg, min(i, a.L1 - 1), L2, lane, gr);
            const float rl = row_ok ? log_norm(scalar_load(rst + i), scalar_load(rst + a.L1 + i)) : INFINITY;
            row_q<CH>(y, gr, r, rl, row_ok, lane, l2, L2, a.sc, lcl, row_ok && l2 == 4 * kWave * CH);
            acc_row<CH>(lacc + wave * kMaxCols, lane, L2, gr, j == 0);
        }
        __syncthreads();
        if (2 * t < L2) {
            const float2* pa = reinterpret_cast<const float2*>(lacc);
            float2 s = pa[t];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) {
                const float2 v = pa[w * (kMaxCols / 2) + t];
                s.x += v.x;
                s.y += v.y;
            }
            s0 += s.x;
            s1 += s.y;
        }
    }
    ldc[2 * t] = s0;
    ldc[2 * t + 1] = s1;
    if (own && 2 * t >= kOwn * m && 2 * t < kOwn * (m + 1)) {
        unsigned long long* r = res_row(a.x, g, p);
        res::publish(r + 2 * t, s0, tag, local);
        res::publish(r + 2 * t + 1, s1, tag, local);
    }
    __syncthreads();
}

template <int CH, bool FW>
__global__ __launch_bounds__(kThreads, 1) void bwd_kernel(BwdArgs1 a) {
    using R = Row<4, CH>;
    const int L2 = FW ? 4 * kWave * CH : a.L2;  // full-width rows: a constant
    constexpr int PL = R::PL;
    __shared__ float rsv[kMembers][kOwn + 1];
    __shared__ __align__(16) float lcl[kMaxCols];  // column log-normalisers
    __shared__ __align__(16) float ldc[kMaxCols];
    // every wave's grad_out rows of the element (loaded during the previous
    // element's exchange); once phase A has read them, the first kWaves rows'
    // worth holds the waves' column partials for the fold
    __shared__ __align__(16) float pre[kWaves * kPreRows * kMaxCols];
    float* const lacc = pre;
    __shared__ int flag;
    __shared__ __align__(16) int votes[kWaves];
    __shared__ int rsflag[kPollWaves];  // (element + 1) << 1 | failed, per polling wave
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int t = threadIdx.x;
    const int G = a.x.groups;
    const int g = blockIdx.x % G;
    const int m = blockIdx.x / G;
    const int n = (a.B - g + G - 1) / G;
    if (n <= 0) return;
    const bool never = a.x.wait_ticks < 0;
    const unsigned tag0 = a.x.epoch << kStageBits;
    if (t == 0) res::publish(xcc_word(a.x, g, m), __int_as_float(res::xcc_id()), tag0);
    if (wave == kWaves - 1) check_group_xcd(a.x, g, tag0, never, &flag);
    if (t < kPollWaves) rsflag[t] = 0;  // read after the first element's barriers
    const int row0 = m * kRowsPerMember + wave * kRowsPerWave;
    float Yv[kRowsPerWave][PL], Gv[kRowsPerWave][PL];
    const size_t elem = size_t(a.L1) * L2;
    const unsigned pre0 = unsigned(uintptr_t((__attribute__((address_space(3))) float*)(pre)));
    {
        // this wave's grad_out rows into LDS (as every later element's), then
        // the sim rows into registers; the LDS rows have landed once at most
        // the 4 CH register-row loads issued after them are outstanding
        const v4u rgw = element_words(a.grad_out, elem, g);
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j)
            load_row_lds<CH>(rgw, min(row0 + j, a.L1 - 1), L2, lane,
                             pre0 + unsigned(wave * kPreRows + j) * kMaxCols * 4u);
        const auto ry = element_rsrc(a.sim, elem, g);
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) load_row<CH>(ry, min(row0 + j, a.L1 - 1), L2, lane, Yv[j]);
        asm volatile("" ::: "memory");  // every load above is issued before the wait
        constexpr unsigned vm = 4 * CH;
        static_assert(vm < 64, "vmcnt field");
        __builtin_amdgcn_s_waitcnt((vm & 15u) | ((vm >> 4) << 14) | 0x0f70u);
    }
    // The next element's grad_out rows of every wave into LDS, by the
    // non-polling waves (each loads two waves' rows)
    auto prefetch = [&](int kn) {
        if (wave >= kPollWaves) {
            const v4u rg = element_words(a.grad_out, elem, g + G * kn);
            const int ln = lane_now();
            constexpr int per = kWaves / (kWaves - kPollWaves);
#pragma unroll
            for (int q = 0; q < per; ++q) {
                const int tw = (wave - kPollWaves) * per + q;
#pragma unroll
                for (int j = 0; j < kRowsPerWave; ++j) {
                    const int i = m * kRowsPerMember + tw * kRowsPerWave + j;
                    load_row_lds<CH>(rg, min(i, a.L1 - 1), L2, ln, pre0 + unsigned(tw * kPreRows + j) * kMaxCols * 4u);
                }
            }
        }
    };
    // column log-normalisers of an element, two columns per thread
    auto col_norm_of = [&](int e, int t) {
        float2 v = make_float2(INFINITY, INFINITY);
        if (2 * t < L2) {
            const float* cst = a.col_stats + size_t(e) * 2 * L2;
            v = make_float2(log_norm(cst[2 * t], cst[L2 + 2 * t]), log_norm(cst[2 * t + 1], cst[L2 + 2 * t + 1]));
        }
        return v;
    };
    float2 ncl = col_norm_of(g, t);
    bool local = false;  // set at element 0's first barrier from the check's flag
    for (int k = 0; k < n; ++k) {
        // thread indices re-formed per element (see lane_now)
        const int lane = lane_now();
        const int t = wave * kWave + lane;
        const int e = g + G * k;
        const unsigned tag = tag0 | unsigned(k + 1);
        const int p = k & 1;
        int l1, l2;
        scalar_extent(a.lengths, e, a.L1, L2, l1, l2);
        reinterpret_cast<float2*>(lcl)[t] = ncl;
        __syncthreads();
        // ---- phase A: (y, g) -> (c, t) and the column-dot partials (in
        // registers: 0 + q of row 0 + ... + q of row 3, acc_row's order)
        const float* rst = a.row_stats + size_t(e) * 2 * a.L1;
        float part[PL];
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) {
            const int i = row0 + j;
            const bool row_ok = i < l1;
            const float rl = row_ok ? log_norm(scalar_load(rst + i), scalar_load(rst + a.L1 + i)) : INFINITY;
            __builtin_amdgcn_sched_barrier(0);  // one row at a time: bounded live ranges
            {  // grad_out from LDS (loaded during the previous element's exchange)
                const float* src = pre + (wave * kPreRows + j) * kMaxCols + 4 * lane;
#pragma unroll
                for (int kk = 0; kk < CH; ++kk) {
                    const float4 v = *reinterpret_cast<const float4*>(src + kk * 256);
                    Gv[j][4 * kk + 0] = v.x;
                    Gv[j][4 * kk + 1] = v.y;
                    Gv[j][4 * kk + 2] = v.z;
                    Gv[j][4 * kk + 3] = v.w;
                }
            }
            float r[PL];
            row_q<CH>(Yv[j], Gv[j], r, rl, row_ok, lane, l2, L2, a.sc, lcl, row_ok && l2 == 4 * kWave * CH);
#pragma unroll
            for (int qq = 0; qq < PL; ++qq) part[qq] = (j == 0 ? 0.0f : part[qq]) + Gv[j][qq];
            float dl = 0.0f;
#pragma unroll
            for (int qq = 0; qq < PL; ++qq) dl += Gv[j][qq];
            const float dr = wave_sum(dl);
            // t formed here: without the asm the compiler sinks this update
            // past the exchange into phase B, keeping r and q both live there
            // (the register file then overflows and spills)
#pragma unroll
            for (int qq = 0; qq < PL; ++qq) {
                Gv[j][qq] = fmaf(-dr, r[qq], 2.0f * Gv[j][qq]);
                asm volatile("" : "+v"(Gv[j][qq]));
            }
        }
        // ---- fold the waves, publish this member's column partials (the
        // partials go where the rows were, once every wave has read its rows)
        lds_barrier();
        R::store(lacc + wave * kMaxCols, lane, L2, part);
        __syncthreads();
        if (k == 0) local = flag != 0 && a.x.local_ok;
        {
            float2 s = make_float2(0.0f, 0.0f);
            if (2 * t < L2) {
                const float2* pa = reinterpret_cast<const float2*>(lacc);
                s = pa[t];
#pragma unroll
                for (int w = 1; w < kWaves; ++w) {
                    const float2 v = pa[w * (kMaxCols / 2) + t];
                    s.x += v.x;
                    s.y += v.y;
                }
            }
            unsigned long long* dst = part_row(a.x, g, p, m) + 2 * t;
            res::publish(dst, s.x, tag, local);
            res::publish(dst + 1, s.y, tag, local);
        }
        const long long deadline = now_ticks() + a.x.wait_ticks;
        const bool real = k + 1 < n;
        // ---- the non-polling waves: the next element's grad_out rows into
        // LDS, once every wave has read the partials there
        lds_barrier();
        if (real) prefetch(k + 1);
        // ---- the polling waves: reduce-scatter, thread t < 256 reads members
        // 4h .. 4h + 3 (h = t / 32) of column 32m + t % 32; then the owner's
        // sums and the all-gather.  The polling waves meet through LDS flags,
        // not a workgroup barrier: the other waves are still issuing their
        // loads, which takes microseconds while HBM is busy.
        int fails = 0;  // bit 1: a reduce-scatter wait expired; bit 0: an all-gather wait
        if (wave < kPollWaves) {
            const int c = t & (kOwn - 1);
            const int h = t >> 5;
            unsigned long long* const w[4] = {
                part_row(a.x, g, p, 4 * h) + kOwn * m + c, part_row(a.x, g, p, 4 * h + 1) + kOwn * m + c,
                part_row(a.x, g, p, 4 * h + 2) + kOwn * m + c, part_row(a.x, g, p, 4 * h + 3) + kOwn * m + c};
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const bool ok = poll4(w, tag, deadline, never, v);
#pragma unroll
            for (int i = 0; i < 4; ++i) rsv[4 * h + i][c] = v[i];
            const int mine = ((k + 1) << 1) | (__ballot(!ok) != 0 ? 1 : 0);
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's rsv values are written
            __hip_atomic_store(&rsflag[wave], mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll 1
            for (int q = 0; q < kPollWaves; ++q) {
                int f;
                do {
                    f = __hip_atomic_load(&rsflag[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                } while ((f >> 1) != k + 1);
                fails |= (f & 1) << 1;
            }
            asm volatile("" ::: "memory");  // rsv is read after the flags
            if (!fails) {
                if (t < kOwn) {
                    float s = 0.0f;
#pragma unroll 8
                    for (int q = 0; q < kMembers; ++q) s += rsv[q][t];
                    res::publish(res_row(a.x, g, p) + kOwn * m + t, s, tag, local);
                }
                // all-gather: thread t < 256 reads columns 4t .. 4t + 3
                unsigned long long* r = res_row(a.x, g, p) + 4 * t;
                unsigned long long* const wr[4] = {r, r + 1, r + 2, r + 3};
                float u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                const bool ok2 = poll4(wr, tag, deadline, never, u);
                *reinterpret_cast<float4*>(ldc + 4 * t) = make_float4(u[0], u[1], u[2], u[3]);
                fails |= __ballot(!ok2) != 0 ? 1 : 0;
            }
        }
        fails = block_or(fails, votes, wave);
        if (fails) {
            // the fallback folds through the rows' LDS: the loads into it
            // land first, and are issued again after it
            if (wave >= kPollWaves) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
            bwd_fallback<CH, FW>(a, e, l1, l2, g, m, p, tag, local, (fails & 2) != 0, lacc, lcl, ldc, wave);
            if (real) prefetch(k + 1);
        }
        // ---- phase B; each row's sim is refilled with the next element's
        // (its grad_out rows are already on their way to LDS)
        if (wave >= kPollWaves) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the prefetch has landed
        const int en = g + G * (real ? k + 1 : k);
        ncl = col_norm_of(en, t);
        const auto ro = element_rsrc(a.grad_sim, elem, e);
        const auto ry = element_rsrc(a.sim, elem, en);
        // One row at a time, its loads after its stores (scheduling barriers):
        // loads hoisted ahead into fresh registers would raise the register
        // count past the file and spill, and a spill reload waits for every
        // store and load the wave has in flight.
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            const int i = row0 + j;
            float o[PL];
            const int z = fresh(0);  // column values read per row (see row_q)
#pragma unroll
            for (int kk = 0; kk < CH; ++kk) {
                float dc[4];
                R::chunk(ldc + z, lane, kk, L2, dc);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int ee = 4 * kk + q;
                    o[ee] = fmaf(-dc[q], Yv[j][ee], Gv[j][ee]) * a.inv_T;
                }
            }
            // the next element's row first: its load waits on HBM, the store
            // can drain behind it
            const int ir = real ? min(i, a.L1 - 1) : 0;
            load_row<CH>(ry, ir, L2, lane, Yv[j]);
            if (i < a.L1) store_row<CH>(ro, i, L2, lane, o);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace onepass
}  // namespace bidi
}  // namespace dot_amd
