// Bidirectional softmax for rows longer than a wave holds in registers
// (L2 > 4096): the sweeps of bidi_kernels.cuh on strips x chunks tiles.
//
// Workgroup (s, c) of batch element b owns rows [s*rows, (s+1)*rows) and
// columns [c*kChunk, (c+1)*kChunk).  Row statistics and row dots come out as
// per-chunk partials in a [B, nchunks, L1] plane and are folded in a fixed
// order by one wave per row; column statistics and column dots keep the
// [B, nstrips, L2] partial layout that fwd_col_combine and column_fold read.
// The reference loops a block over any row length (kernels.cu:90-139,
// :153-202); its column kernels walk columns with stride L2.
#pragma once

#include "bidi_kernels.cuh"
#include "tile.cuh"

#pragma clang fp contract(off)

namespace dot_amd {
namespace bidi {
namespace wide_rows {

using dot_amd::wide::kChunk;
using dot_amd::wide::Tile;
using dot_amd::wide::tile_of_block;

// Valid columns of a chunk: those below the element's l2.
__device__ __forceinline__ int chunk_valid(int l2, const Tile& t) { return max(0, min(l2 - t.c0, t.nc)); }

struct Args {
    FwdArgs f;         // forward: statistics planes, strip partials, outputs
    BwdArgs g;         // backward: dots, strip partials, gradient
    float2* rpart;     // [B, nchunks, L1]: row (max, sum) partials (forward)
    float* dpart;      // [B, nchunks, L1]: row dot partials (backward)
    int B, nchunks;
};

// Row statistics partials (base-2 max and sum of 2^(y2 - max) over the chunk)
// and per-strip column states of the chunk's columns.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void fwd_stats(Args w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const FwdArgs& a = w.f;
    extern __shared__ __align__(16) float lds[];
    const Tile tl = tile_of_block(w.nchunks, a.L2);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const int nv = chunk_valid(l2, tl);
    const float sc = a.inv_T * kLog2E;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, l1);
    float cm[R::PL], cs[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        cm[e] = -FLT_MAX;
        cs[e] = 0.0f;
    }
    float2* part = w.rpart + (size_t(b) * w.nchunks + tl.c) * a.L1;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float y[R::PL];
        R::load(a.sim + (size_t(b) * a.L1 + i) * a.L2 + tl.c0, lane, tl.nc, y, 0.0f);
        float ml = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            y[e] = R::valid(lane, e, nv) ? y[e] * sc : -INFINITY;
            ml = fmaxf(ml, y[e]);
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
        if (lane == 0) part[i] = make_float2(rm, rs);
    }
    block_column_combine_lse<VEC, CH>(cm, cs, lds, tl.nc);
    if (wave == 0) {
        const size_t off = (size_t(b) * a.nstrips + tl.s) * a.L2 + tl.c0;
        R::store(a.part_m + off, lane, tl.nc, cm);
        R::store(a.part_s + off, lane, tl.nc, cs);
    }
}

// Row statistics of the valid rows from the chunk partials (base-2 merge in
// chunk order); one wave per row.
static __global__ __launch_bounds__(kBlock) void fwd_row_stats(Args w) {
    const FwdArgs& a = w.f;
    const size_t row = size_t(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
    if (row >= size_t(w.B) * a.L1) return;
    const int b = int(row / a.L1), i = int(row % a.L1);
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    if (i >= l1) return;
    const int lane = threadIdx.x % kWave;
    const float2* p = w.rpart + size_t(b) * w.nchunks * a.L1 + i;
    float m = -FLT_MAX, s = 0.0f;
    for (int c = lane; c < w.nchunks; c += kWave) {
        const float2 q = p[size_t(c) * a.L1];
        lse_merge2(m, s, q.x, q.y);
    }
    const float M = wave_max(m);
    const float S = wave_sum(s * __builtin_amdgcn_exp2f(m - M));
    if (lane == 0) {
        float* rs = a.row_stats + size_t(b) * 2 * a.L1;
        rs[i] = M;
        rs[a.L1 + i] = S;
    }
}

// r, c, out for one chunk of the strip's rows (as fwd_write); zero rows and
// columns outside the valid region.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void fwd_write(Args w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const FwdArgs& a = w.f;
    extern __shared__ __align__(16) float lds[];  // column max | 1 / column sum, kChunk each
    const Tile tl = tile_of_block(w.nchunks, a.L2);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const int nv = chunk_valid(l2, tl);
    const float sc = a.inv_T * kLog2E;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.L1);
    float* lcm = lds;
    float* lics = lds + kChunk;
    load_col_stats(a.col_stats + size_t(b) * 2 * a.L2 + tl.c0, a.L2, tl.nc, lcm, lics);
    __syncthreads();
    const float* rstat = a.row_stats + size_t(b) * 2 * a.L1;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (size_t(b) * a.L1 + i) * a.L2 + tl.c0;
        float o[R::PL], rr[R::PL], cc[R::PL];
        if (i < l1) {
            float y[R::PL];
            R::load(a.sim + off, lane, tl.nc, y, 0.0f);
            const float rm = rstat[i];
            const float rsum = rstat[a.L1 + i];
            const float irs = rsum > 0.0f ? 1.0f / rsum : 0.0f;
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float cm[VEC], ics[VEC];
                R::chunk(lcm, lane, k, tl.nc, cm);
                R::chunk(lics, lane, k, tl.nc, ics);
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    const int e = k * VEC + q;
                    const bool ok = R::valid(lane, e, nv);
                    const float y2 = y[e] * sc;
                    rr[e] = ok ? __builtin_amdgcn_exp2f(y2 - rm) * irs : 0.0f;
                    cc[e] = ok ? __builtin_amdgcn_exp2f(y2 - cm[q]) * ics[q] : 0.0f;
                    o[e] = ok ? __builtin_amdgcn_sqrtf(fmaf(rr[e], cc[e], kEps)) : 0.0f;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < R::PL; ++e) o[e] = rr[e] = cc[e] = 0.0f;
        }
        R::store_stream(a.out + off, lane, tl.nc, o);
        if (a.row_sm) R::store_stream(a.row_sm + off, lane, tl.nc, rr);
        if (a.col_sm) R::store_stream(a.col_sm + off, lane, tl.nc, cc);
    }
}

// r, c and d = g / (2 out) for one row chunk, from the forward's buffers or
// recomputed from the statistics (as BwdRow::get); 0 outside the valid region.
template <int VEC, int CH, bool RECOMPUTE>
__device__ __forceinline__ void bwd_terms(const BwdArgs& a, size_t off, int lane, int nc, int nv, float rm,
                                          float irs, const float* lcm, const float* lics,
                                          float (&y)[VEC * CH], float (&r)[VEC * CH], float (&c)[VEC * CH],
                                          float (&d)[VEC * CH]) {
    using R = Row<VEC, CH>;
    float g[R::PL];
    R::load(a.sim + off, lane, nc, y, 0.0f);
    R::load(a.grad_out + off, lane, nc, g, 0.0f);
    if constexpr (RECOMPUTE) {
        const float sc = a.inv_T * kLog2E;
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            float cm[VEC], ics[VEC];
            R::chunk(lcm, lane, k, nc, cm);
            R::chunk(lics, lane, k, nc, ics);
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
                const int e = k * VEC + q;
                const bool ok = R::valid(lane, e, nv);
                const float y2 = y[e] * sc;
                r[e] = ok ? __builtin_amdgcn_exp2f(y2 - rm) * irs : 0.0f;
                c[e] = ok ? __builtin_amdgcn_exp2f(y2 - cm[q]) * ics[q] : 0.0f;
                const float o = __builtin_amdgcn_sqrtf(fmaf(r[e], c[e], kEps));
                d[e] = ok ? (g[e] * 0.5f) * __builtin_amdgcn_rcpf(o) : 0.0f;
            }
        }
    } else {
        float o[R::PL];
        R::load(a.row_sm + off, lane, nc, r, 0.0f);
        R::load(a.col_sm + off, lane, nc, c, 0.0f);
        R::load(a.out + off, lane, nc, o, 0.0f);
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const bool ok = R::valid(lane, e, nv) && o[e] > kEps;
            d[e] = ok ? (g[e] * 0.5f) * __builtin_amdgcn_rcpf(o[e]) : 0.0f;
        }
    }
}

// Row statistics and column statistics of a chunk into LDS (recompute mode).
__device__ __forceinline__ void bwd_stats_to_lds(const BwdArgs& a, int b, const Tile& tl, float* lcm,
                                                 float* lics) {
    load_col_stats(a.col_stats + size_t(b) * 2 * a.L2 + tl.c0, a.L2, tl.nc, lcm, lics);
}

__device__ __forceinline__ void row_stat(const BwdArgs& a, int b, int i, float& rm, float& irs) {
    const float* rs = a.row_stats + size_t(b) * 2 * a.L1;
    rm = rs[i];
    const float s = rs[a.L1 + i];
    irs = s > 0.0f ? 1.0f / s : 0.0f;
}

// Row dot partials sum_j (d c) r over the chunk and the chunk's column partials
// of (d r) c over the strip.
template <int VEC, int CH, bool RECOMPUTE>
__global__ __launch_bounds__(kBlock) void bwd_dots(Args w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const BwdArgs& a = w.g;
    extern __shared__ __align__(16) float lds[];  // column stats 2 kChunk | column combine 2 kChunk + 8
    const Tile tl = tile_of_block(w.nchunks, a.L2);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const int nv = chunk_valid(l2, tl);
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, l1);
    float* lcm = lds;
    float* lics = lds + kChunk;
    if constexpr (RECOMPUTE) bwd_stats_to_lds(a, b, tl, lcm, lics);
    __syncthreads();
    float* part = w.dpart + (size_t(b) * w.nchunks + tl.c) * a.L1;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float rm = 0.0f, irs = 0.0f;
        if constexpr (RECOMPUTE) row_stat(a, b, i, rm, irs);
        float y[R::PL], r[R::PL], c[R::PL], d[R::PL];
        bwd_terms<VEC, CH, RECOMPUTE>(a, (size_t(b) * a.L1 + i) * a.L2 + tl.c0, lane, tl.nc, nv, rm, irs,
                                      lcm, lics, y, r, c, d);
        float dl = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            dl = fmaf(d[e] * c[e], r[e], dl);
            acc[e] = fmaf(d[e] * r[e], c[e], acc[e]);
        }
        const float dr = wave_sum(dl);
        if (lane == 0) part[i] = dr;
    }
    block_column_combine<VEC, CH>(acc, lds + 2 * kChunk, tl.nc);
    if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + tl.s) * a.L2 + tl.c0, lane, tl.nc, acc);
}

// dot_r of the valid rows from the chunk partials; one wave per row.
static __global__ __launch_bounds__(kBlock) void bwd_row_dots(Args w) {
    const BwdArgs& a = w.g;
    const size_t row = size_t(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
    if (row >= size_t(w.B) * a.L1) return;
    const int b = int(row / a.L1), i = int(row % a.L1);
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    if (i >= l1) return;
    const float t = dot_amd::wide::fold_sum(w.dpart + size_t(b) * w.nchunks * a.L1 + i, a.L1, w.nchunks);
    if (threadIdx.x % kWave == 0) a.dot_r[size_t(b) * a.L1 + i] = t;
}

// grad = ((d c - dot_r) r + (d r - dot_c) c) / tau for one chunk, 0 outside
// the valid region, and per-tile sums of grad * sim; tau_partial is [B, gridDim.x].
template <int VEC, int CH, bool RECOMPUTE>
__global__ __launch_bounds__(kBlock) void bwd_write(Args w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const BwdArgs& a = w.g;
    __shared__ float scratch[kWavesPerBlock];
    extern __shared__ __align__(16) float lds[];  // column stats 2 kChunk | column dots kChunk
    const Tile tl = tile_of_block(w.nchunks, a.L2);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    int l1, l2;
    valid_extent(a.lengths, b, a.L1, a.L2, l1, l2);
    const int nv = chunk_valid(l2, tl);
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.L1);
    float* lcm = lds;
    float* lics = lds + kChunk;
    float* ldc = lds + 2 * kChunk;
    if constexpr (RECOMPUTE) bwd_stats_to_lds(a, b, tl, lcm, lics);
    for (int j = threadIdx.x; j < tl.nc; j += kBlock) ldc[j] = a.dot_c[size_t(b) * a.L2 + tl.c0 + j];
    __syncthreads();
    float tacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (size_t(b) * a.L1 + i) * a.L2 + tl.c0;
        float gs[R::PL];
        if (i < l1) {
            float rm = 0.0f, irs = 0.0f;
            if constexpr (RECOMPUTE) row_stat(a, b, i, rm, irs);
            float y[R::PL], r[R::PL], c[R::PL], d[R::PL];
            bwd_terms<VEC, CH, RECOMPUTE>(a, off, lane, tl.nc, nv, rm, irs, lcm, lics, y, r, c, d);
            const float dr = a.dot_r[size_t(b) * a.L1 + i];
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                float dc[VEC];
                R::chunk(ldc, lane, k, tl.nc, dc);
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    const int e = k * VEC + q;
                    const bool valid = R::valid(lane, e, nv);
                    const float tt = (d[e] * c[e] - dr) * r[e] + (d[e] * r[e] - dc[q]) * c[e];
                    gs[e] = valid ? tt * a.inv_T : 0.0f;
                    if (a.tau_partial) tacc = valid ? fmaf(gs[e], y[e], tacc) : tacc;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < R::PL; ++e) gs[e] = 0.0f;
        }
        R::store_stream(a.grad_sim + off, lane, tl.nc, gs);
    }
    if (a.tau_partial) {
        const float tsum = block_reduce<kWavesPerBlock>(wave_sum(tacc), scratch, OpSum{});
        if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + blockIdx.x] = tsum;
    }
}

}  // namespace wide_rows
}  // namespace bidi
}  // namespace dot_amd
