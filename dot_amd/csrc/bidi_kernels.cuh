// Bidirectional softmax device kernels.
//
// out = sqrt(1e-9 + r * c) with r the row softmax and c the column softmax of
// sim / tau inside the valid region [0, L1_b) x [0, L2_b), 0 outside
// (src/bidirectional_softmax/kernels.cu:90-242).  The forward is two sweeps:
// a statistics sweep (row max/sum per wave; per-column online max/sum over the
// strip, merged across strips) and a write sweep.  The backward is two sweeps
// too: row and column dot products of q = d * r * c, then the gradient.
// Statistics are stored as planes: row_stats [B, 2, L1] (max plane, then sum
// plane) and col_stats [B, 2, L2], maxima in base-2 units (see below).
#pragma once

#include <cfloat>
#include <cstdint>

#include "row.cuh"

// No automatic FMA contraction here: every kernel forms y2 = sim * sc with the
// same rounding, so the entry that attains a stored maximum gives exactly
// 2^(y2 - max) = 1; a contracted fma(sim, sc, -max) would not.
#pragma clang fp contract(off)

namespace dot_amd {
namespace bidi {

constexpr float kEps = 1.0e-9f;  // kernels.cu:29

__device__ __forceinline__ void valid_extent(const int32_t* lengths, int b, int L1, int L2, int& l1,
                                             int& l2) {
    if (!lengths) {  // no lengths: every element is full
        l1 = L1;
        l2 = L2;
        return;
    }
    l1 = min(max(lengths[2 * b], 0), L1);
    l2 = min(max(lengths[2 * b + 1], 0), L2);
}

// Merge of two column states kept in base 2 (sum = s * 2^m).
__device__ __forceinline__ void lse_merge2(float& m, float& s, float m2, float s2) {
    const float M = fmaxf(m, m2);
    s = s * __builtin_amdgcn_exp2f(m - M) + s2 * __builtin_amdgcn_exp2f(m2 - M);
    m = M;
}

// Fold the base-2 (m, s) column states of the 4 waves into wave 0 in the fixed order
// (w0 + w2) + (w1 + w3).  `lds` holds 2*N floats; every thread must call it.
template <int VEC, int CH>
__device__ __forceinline__ void block_column_combine_lse(float (&m)[VEC * CH], float (&s)[VEC * CH],
                                                         float* lds, int N) {
    using R = Row<VEC, CH>;
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform: scalar row loads
    // (source wave, destination wave) per round
    constexpr int kRounds[3][2] = {{3, 1}, {2, 0}, {1, 0}};
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        __syncthreads();
        if (wave == kRounds[r][0]) {
            R::store(lds, lane, N, m);
            R::store(lds + N, lane, N, s);
        }
        __syncthreads();
        if (wave == kRounds[r][1]) {
            float m2[R::PL], s2[R::PL];
            R::load(lds, lane, N, m2, -FLT_MAX);
            R::load(lds + N, lane, N, s2, 0.0f);
#pragma unroll
            for (int e = 0; e < R::PL; ++e) lse_merge2(m[e], s[e], m2[e], s2[e]);
        }
    }
}

struct FwdArgs {
    const float* sim;
    const int32_t* lengths;
    float inv_T;
    int B, L1, L2, rows, nstrips;
    float* row_stats;    // [B,2,L1]
    float* col_stats;    // [B,2,L2]
    float* part_m;       // [B,nstrips,L2]
    float* part_s;       // [B,nstrips,L2]
    float* out;          // [B,L1,L2]
    float* row_sm;       // or null
    float* col_sm;       // or null
};

// Exponentials run in base 2 on y2 = sim * (inv_T * log2(e)): exp(y - m) =
// 2^(y2 - m2).  The statistics keep the maxima in that unit (m2 = max y2) and
// the sums unchanged (sum of exp(y - max)); every kernel forms y2 with the
// same expression, so the entry that attains a maximum gives exactly 2^0 = 1.

// Lanes past the valid columns hold -inf (their exponentials are 0).  `full`
// (every lane of every chunk is a valid column) lets the loops skip the test.
template <class R>
__device__ __forceinline__ float masked(float y2, bool full, int lane, int e, int l2) {
    return (full || R::valid(lane, e, l2)) ? y2 : -INFINITY;
}

// Row statistics (kernels.cu:90-139: max of sim*inv_T, sum of safe_exp(y - max))
// and per-strip column statistics (kernels.cu:153-202) in one read of sim.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void fwd_stats(FwdArgs a) {
    using R = Row<VEC, CH>;
    extern __shared__ __align__(16) float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform: scalar row loads
    const int st = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const bool full = l2 == kWave * R::PL;
    const float sc = a.inv_T * kLog2E;
    const int r0 = st * a.rows;
    const int r1 = min(r0 + a.rows, l1);
    float cm[R::PL], cs[R::PL];  // column state in base 2: sum = cs * 2^cm
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        cm[e] = -FLT_MAX;
        cs[e] = 0.0f;
    }
    float* rmax = a.row_stats + size_t(b) * 2 * a.L1;
    float* rsum = rmax + a.L1;
    const float* base = a.sim + size_t(b) * a.L1 * a.L2;
    struct Buf {
        float v[R::PL];
    };
    auto load = [&](int i, Buf& t) { R::load_clamped(base + size_t(i) * a.L2, lane, a.L2, t.v, 0.0f); };
    pipelined_rows<Buf>(r0 + wave, r1, kWavesPerBlock, load, [&](int i, Buf& t) {
        float(&y)[R::PL] = t.v;
        float ml = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            y[e] = masked<R>(y[e] * sc, full, lane, e, l2);
            ml = fmaxf(ml, y[e]);
            // online column state: one exponential per element
            const float d = y[e] - cm[e];
            const float x = __builtin_amdgcn_exp2f(-fabsf(d));
            const bool gt = d > 0.0f;
            cs[e] = gt ? fmaf(cs[e], x, 1.0f) : cs[e] + x;
            cm[e] = gt ? y[e] : cm[e];
        }
        const float rm = wave_max(ml);
        float sl = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) sl += __builtin_amdgcn_exp2f(y[e] - rm);
        const float rs = wave_sum(sl);
        // every lane stores the same value: no branch, so the look-ahead's
        // wait counts stay exact
        rmax[i] = rm;
        rsum[i] = rs;
    });
    block_column_combine_lse<VEC, CH>(cm, cs, lds, a.L2);
    if (wave == 0) {
        const size_t off = (size_t(b) * a.nstrips + st) * a.L2;
        R::store(a.part_m + off, lane, a.L2, cm);
        R::store(a.part_s + off, lane, a.L2, cs);
    }
}

// Column statistics: merge the strips' base-2 states.  A block takes
// kFoldCols columns; its kFoldLanes lanes per column merge strips
// lane, lane + kFoldLanes, ... in order, then a fixed halving tree in LDS
// merges the lanes, so every column sees the same order on every run.
constexpr int kFoldCols = 16;
constexpr int kFoldLanes = kBlock / kFoldCols;  // 16

static __global__ __launch_bounds__(kBlock) void fwd_col_combine(FwdArgs a) {
    __shared__ float sm_m[kFoldLanes][kFoldCols], sm_s[kFoldLanes][kFoldCols];
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int jj = threadIdx.x % kFoldCols;
    const int sl = threadIdx.x / kFoldCols;
    const int j = blockIdx.x * kFoldCols + jj;
    float m = -FLT_MAX, s = 0.0f;
    if (j < a.L2) {
        const size_t base = size_t(b) * a.nstrips * a.L2 + j;
        for (int k = sl; k < a.nstrips; k += kFoldLanes)
            lse_merge2(m, s, a.part_m[base + size_t(k) * a.L2], a.part_s[base + size_t(k) * a.L2]);
    }
    sm_m[sl][jj] = m;
    sm_s[sl][jj] = s;
#pragma unroll
    for (int half = kFoldLanes / 2; half >= 1; half /= 2) {
        __syncthreads();
        if (sl < half) {
            lse_merge2(m, s, sm_m[sl + half][jj], sm_s[sl + half][jj]);
            sm_m[sl][jj] = m;
            sm_s[sl][jj] = s;
        }
    }
    if (sl == 0 && j < a.L2) {
        float* cmax = a.col_stats + size_t(b) * 2 * a.L2;
        cmax[j] = m;
        cmax[a.L2 + j] = s;
    }
}

// Column sums of the strips' partial rows, in the same fixed order as
// fwd_col_combine.
static __global__ __launch_bounds__(kBlock) void column_fold(const float* partial, int nstrips, int B, int N,
                                                             float* out) {
    __shared__ float sm[kFoldLanes][kFoldCols];
    const int b = batch_of_block();
    if (b >= B) return;
    const int jj = threadIdx.x % kFoldCols;
    const int sl = threadIdx.x / kFoldCols;
    const int j = blockIdx.x * kFoldCols + jj;
    float s = 0.0f;
    if (j < N) {
        const size_t base = size_t(b) * nstrips * N + j;
        for (int k = sl; k < nstrips; k += kFoldLanes) s += partial[base + size_t(k) * N];
    }
    sm[sl][jj] = s;
#pragma unroll
    for (int half = kFoldLanes / 2; half >= 1; half /= 2) {
        __syncthreads();
        if (sl < half) {
            s += sm[sl + half][jj];
            sm[sl][jj] = s;
        }
    }
    if (sl == 0 && j < N) out[size_t(b) * N + j] = s;
}

// Column max and reciprocal column sum of one batch element into LDS, shared
// by the block's waves (registers would hold them for the whole kernel and cost
// occupancy).  The caller places the barrier before the first read.
__device__ __forceinline__ void load_col_stats(const float* cstat, int L2, int n, float* lcm, float* lics) {
    // n columns from cstat (a column max plane, its sum plane L2 floats later)
    for (int j = threadIdx.x; j < n; j += kBlock) {
        lcm[j] = cstat[j];
        const float cs = cstat[L2 + j];
        lics[j] = cs > 0.0f ? 1.0f / cs : 0.0f;
    }
}

__device__ __forceinline__ void load_col_stats(const float* cstat, int L2, float* lcm, float* lics) {
    load_col_stats(cstat, L2, L2, lcm, lics);
}

// Row max and reciprocal row sum of the strip's valid rows [r0, r1) into LDS
// (read there, per-row global loads would queue behind the rows loaded ahead).
// The caller places the barrier before the first read.
__device__ __forceinline__ void load_row_stats(const float* rstat, int L1, int r0, int r1, float* lrm,
                                               float* lirs) {
    for (int t = threadIdx.x; t < r1 - r0; t += kBlock) {
        lrm[t] = rstat[r0 + t];
        const float rs = rstat[L1 + r0 + t];
        lirs[t] = rs > 0.0f ? 1.0f / rs : 0.0f;
    }
}

// r = exp(y - rmax) / rsum, c = exp(y - cmax) / csum, out = sqrt(1e-9 + r c);
// zeros outside the valid region (kernels.cu:143-149, :206-212, :216-242).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void fwd_write(FwdArgs a) {
    using R = Row<VEC, CH>;
    // LDS: column max (base 2) L2 | 1 / column sum L2 | row max rows | 1 / row sum rows
    extern __shared__ __align__(16) float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int b = batch_of_block();
    if (b >= a.B) return;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const bool full = l2 == kWave * R::PL;
    const float sc = a.inv_T * kLog2E;
    const int r0 = blockIdx.x * a.rows;
    const int r1 = min(r0 + a.rows, a.L1);
    const int rv = min(r1, l1);  // end of the valid rows
    float* lcm = lds;
    float* lics = lds + a.L2;
    float* lrm = lds + 2 * a.L2;
    float* lirs = lrm + a.rows;
    load_col_stats(a.col_stats + size_t(b) * 2 * a.L2, a.L2, lcm, lics);
    load_row_stats(a.row_stats + size_t(b) * 2 * a.L1, a.L1, r0, rv, lrm, lirs);
    __syncthreads();
    auto write = [&](int i, const float(&o)[R::PL], const float(&rr)[R::PL], const float(&cc)[R::PL]) {
        const size_t off = (size_t(b) * a.L1 + i) * a.L2;
        R::store_stream(a.out + off, lane, a.L2, o);
        if (a.row_sm) R::store_stream(a.row_sm + off, lane, a.L2, rr);
        if (a.col_sm) R::store_stream(a.col_sm + off, lane, a.L2, cc);
    };
    // rows of the valid region, then the zero rows past it
    auto load = [&](int i, RowBuf<R>& t) {
        R::load_clamped(a.sim + (size_t(b) * a.L1 + i) * a.L2, lane, a.L2, t.v, 0.0f);
    };
    pipelined_rows<RowBuf<R>>(r0 + wave, rv, kWavesPerBlock, load, [&](int i, RowBuf<R>& t) {
        const float rm = lrm[i - r0];
        const float irs = lirs[i - r0];
        float o[R::PL], rr[R::PL], cc[R::PL];
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            float cm[VEC], ics[VEC];
            R::chunk(lcm, lane, k, a.L2, cm);
            R::chunk(lics, lane, k, a.L2, ics);
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
                const int e = k * VEC + q;
                const bool ok = full || R::valid(lane, e, l2);
                const float y2 = t.v[e] * sc;
                rr[e] = ok ? __builtin_amdgcn_exp2f(y2 - rm) * irs : 0.0f;
                cc[e] = ok ? __builtin_amdgcn_exp2f(y2 - cm[q]) * ics[q] : 0.0f;
                o[e] = ok ? __builtin_amdgcn_sqrtf(fmaf(rr[e], cc[e], kEps)) : 0.0f;
            }
        }
        write(i, o, rr, cc);
    });
    float z[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) z[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock)
        if (i >= l1) write(i, z, z, z);
}

struct BwdArgs {
    const float* sim;
    const int32_t* lengths;
    float inv_T;
    int B, L1, L2, rows, nstrips;
    const float* grad_out;
    const float* out;      // buffer mode
    const float* row_sm;
    const float* col_sm;
    const float* row_stats;  // recompute mode
    const float* col_stats;
    float* dot_r;          // [B,L1]
    float* dot_c;          // [B,L2]
    float* partial;        // [B,nstrips,L2]
    float* grad_sim;
    float* tau_partial;    // [B,gridDim.x], or null when grad_tau is not requested
};

// For one row: r, c and d = g / (2 out) (kernels.cu:249-274), from the
// forward's buffers or recomputed from the statistics; 0 outside the valid
// region.  In recompute mode out >= sqrt(1e-9) > 1e-9, so the reference's
// out > 1e-9 test always passes.  A row's inputs are loaded into a Buf first
// (sim and grad_out; plus the three buffers in buffer mode), so the kernels can
// load rows ahead.
template <int VEC, int CH, bool RECOMPUTE>
struct BwdRow {
    using R = Row<VEC, CH>;
    static constexpr int kBufPL = RECOMPUTE ? 1 : R::PL;
    struct Buf {
        float y[R::PL], g[R::PL];
        float r[kBufPL], c[kBufPL], o[kBufPL];
    };
    const float* lcm;   // LDS: column max (base 2), L2 floats
    const float* lics;  // LDS: 1 / column sum
    const float* lrm;   // LDS: row max (base 2) of the strip's rows
    const float* lirs;  // LDS: 1 / row sum
    int r0;
    float sc;

    // `lds` holds 2 * L2 + 2 * rows floats; the caller places the barrier
    // before the first get().  [r0, rv) are the strip's valid rows.
    __device__ void init(const BwdArgs& a, int b, float* lds, int r0_, int rv) {
        sc = a.inv_T * kLog2E;
        r0 = r0_;
        float* cm = lds;
        float* ics = lds + a.L2;
        float* rm = lds + 2 * a.L2;
        float* irs = rm + a.rows;
        lcm = cm;
        lics = ics;
        lrm = rm;
        lirs = irs;
        if constexpr (RECOMPUTE) {
            load_col_stats(a.col_stats + size_t(b) * 2 * a.L2, a.L2, cm, ics);
            load_row_stats(a.row_stats + size_t(b) * 2 * a.L1, a.L1, r0, rv, rm, irs);
        }
    }

    __device__ void load(const BwdArgs& a, size_t off, int lane, Buf& t) const {
        R::load_clamped(a.sim + off, lane, a.L2, t.y, 0.0f);
        R::load_clamped(a.grad_out + off, lane, a.L2, t.g, 0.0f);
        if constexpr (!RECOMPUTE) {
            R::load(a.row_sm + off, lane, a.L2, t.r, 0.0f);
            R::load(a.col_sm + off, lane, a.L2, t.c, 0.0f);
            R::load(a.out + off, lane, a.L2, t.o, 0.0f);
        }
    }

    __device__ void get(const BwdArgs& a, int i, int lane, int l2, bool full, const Buf& t,
                        float (&r)[R::PL], float (&c)[R::PL], float (&d)[R::PL]) const {
        if constexpr (RECOMPUTE) {
            const float rm = lrm[i - r0];
            const float irs = lirs[i - r0];
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float cm[VEC], ics[VEC];
                R::chunk(lcm, lane, k, a.L2, cm);
                R::chunk(lics, lane, k, a.L2, ics);
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    const int e = k * VEC + q;
                    const bool ok = full || R::valid(lane, e, l2);
                    const float y2 = t.y[e] * sc;
                    r[e] = ok ? __builtin_amdgcn_exp2f(y2 - rm) * irs : 0.0f;
                    c[e] = ok ? __builtin_amdgcn_exp2f(y2 - cm[q]) * ics[q] : 0.0f;
                    const float o = __builtin_amdgcn_sqrtf(fmaf(r[e], c[e], kEps));
                    d[e] = ok ? (t.g[e] * 0.5f) * __builtin_amdgcn_rcpf(o) : 0.0f;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < R::PL; ++e) {
                r[e] = t.r[e];
                c[e] = t.c[e];
                const bool ok = (full || R::valid(lane, e, l2)) && t.o[e] > kEps;
                d[e] = ok ? (t.g[e] * 0.5f) * __builtin_amdgcn_rcpf(t.o[e]) : 0.0f;
            }
        }
    }
};

// Visits the rows of `src` with loads ahead in recompute mode (two row buffers
// of sim and grad_out); buffer mode, with five arrays per row, visits them
// one at a time.
template <bool RECOMPUTE, class Src, class Body>
__device__ __forceinline__ void bwd_rows(const BwdArgs& a, const Src& src, int b, int i0, int r1, int lane,
                                         Body&& body) {
    using Buf = typename Src::Buf;
    auto load = [&](int i, Buf& t) { src.load(a, (size_t(b) * a.L1 + i) * a.L2, lane, t); };
    if constexpr (RECOMPUTE) {
        pipelined_rows<Buf>(i0, r1, kWavesPerBlock, load, body);
    } else {
        for (int i = i0; i < r1; i += kWavesPerBlock) {
            Buf t;
            load(i, t);
            body(i, t);
        }
    }
}

// Row dots sum_j (d c) r and column partials of (d r) c over the strip
// (kernels.cu:277-354).
template <int VEC, int CH, bool RECOMPUTE>
__global__ __launch_bounds__(kBlock) void bwd_dots(BwdArgs a) {
    using R = Row<VEC, CH>;
    using Src = BwdRow<VEC, CH, RECOMPUTE>;
    // LDS: statistics 2 * L2 + 2 * rows | block_column_combine's 2 * L2 + 8
    extern __shared__ __align__(16) float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int st = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const bool full = l2 == kWave * R::PL;
    const int r0 = st * a.rows;
    const int r1 = min(r0 + a.rows, l1);
    Src src;
    src.init(a, b, lds, r0, r1);
    __syncthreads();
    float* comb = lds + 2 * a.L2 + 2 * a.rows;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    bwd_rows<RECOMPUTE>(a, src, b, r0 + wave, r1, lane, [&](int i, const typename Src::Buf& t) {
        float r[R::PL], c[R::PL], d[R::PL];
        src.get(a, i, lane, l2, full, t, r, c, d);
        float dl = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            dl = fmaf(d[e] * c[e], r[e], dl);
            acc[e] = fmaf(d[e] * r[e], c[e], acc[e]);
        }
        const float dr = wave_sum(dl);
        a.dot_r[size_t(b) * a.L1 + i] = dr;  // every lane stores the same value (no branch)
    });
    block_column_combine<VEC, CH>(acc, comb, a.L2);
    if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + st) * a.L2, lane, a.L2, acc);
}

// grad = ((d c - dot_r) r + (d r - dot_c) c) / tau in the valid region, 0
// elsewhere; per-block sums of grad * sim for grad_tau (kernels.cu:379-411).
template <int VEC, int CH, bool RECOMPUTE>
__global__ __launch_bounds__(kBlock) void bwd_write(BwdArgs a) {
    using R = Row<VEC, CH>;
    using Src = BwdRow<VEC, CH, RECOMPUTE>;
    __shared__ float scratch[kWavesPerBlock];
    // LDS: statistics 2 * L2 + 2 * rows | column dots L2 | row dots rows
    extern __shared__ __align__(16) float lds[];
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int b = batch_of_block();
    if (b >= a.B) return;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const bool full = l2 == kWave * R::PL;
    const int r0 = blockIdx.x * a.rows;
    const int r1 = min(r0 + a.rows, a.L1);
    const int rv = min(r1, l1);
    float* ldc = lds + 2 * a.L2 + 2 * a.rows;
    float* ldr = ldc + a.L2;
    for (int j = threadIdx.x; j < a.L2; j += kBlock) ldc[j] = a.dot_c[size_t(b) * a.L2 + j];
    for (int t = threadIdx.x; t < rv - r0; t += kBlock) ldr[t] = a.dot_r[size_t(b) * a.L1 + r0 + t];
    Src src;
    src.init(a, b, lds, r0, rv);
    __syncthreads();
    float tacc = 0.0f;
    const bool want_tau = a.tau_partial != nullptr;  // null: grad_tau not requested
    auto store = [&](int i, const float(&gs)[R::PL]) {
        R::store_stream(a.grad_sim + (size_t(b) * a.L1 + i) * a.L2, lane, a.L2, gs);
    };
    bwd_rows<RECOMPUTE>(a, src, b, r0 + wave, rv, lane, [&](int i, const typename Src::Buf& t) {
        float r[R::PL], c[R::PL], d[R::PL], gs[R::PL];
        src.get(a, i, lane, l2, full, t, r, c, d);
        const float dr = ldr[i - r0];
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            float dc[VEC];
            R::chunk(ldc, lane, k, a.L2, dc);
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
                const int e = k * VEC + q;
                const bool valid = full || R::valid(lane, e, l2);
                const float tt = (d[e] * c[e] - dr) * r[e] + (d[e] * r[e] - dc[q]) * c[e];
                gs[e] = valid ? tt * a.inv_T : 0.0f;
                if (want_tau) tacc = valid ? fmaf(gs[e], t.y[e], tacc) : tacc;
            }
        }
        store(i, gs);
    });
    float z[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) z[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock)
        if (i >= l1) store(i, z);
    if (want_tau) {
        const float tsum = block_reduce<kWavesPerBlock>(wave_sum(tacc), scratch, OpSum{});
        if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + blockIdx.x] = tsum;
    }
}

}  // namespace bidi
}  // namespace dot_amd
