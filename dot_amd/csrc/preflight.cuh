// Spectral preflight: the contraction estimate behind n_iters='auto'
// (src/sinkhorn/kernels.cu:141-241, dot/sinkhorn.py:860-897).
//
// With P = softmax_row(log_alpha / tau) and v0_j = sin((j+1) 12.9898 +
// (b+1) 78.233) centred and normalised, n_power deflated power iterations
//   u = centre(P v);  v = centre_normalise(P^T u)
// and a last u = centre(P v) give tau_est = ||u|| clamped to [0, 0.999999].
// The reference runs one 1024-thread block per batch element over serial
// O(n m) loops; here every product is a streaming sweep over row strips (the
// Row layout of the Sinkhorn sweeps, P recomputed from log_alpha and the row
// log-sum-exp on load) and the per-element vector work is one block per
// element:
//   spf_lse     row log-sum-exp of log_alpha / tau
//   spf_init    v0, centred and normalised
//   per power iteration:
//     spf_rowdot  u_i = sum_j P_ij v_j, and per-strip sums of u
//     spf_coldot  per-strip column sums of P_ij (u_i - mean u)
//     spf_vfold   v = sum over strips, centred and normalised
//   spf_rowdot, then spf_final: ||u - mean u||.
// Rows longer than kMaxRowLen run the row sweeps over the strips x chunks
// tiles of tile.cuh: each row reduction writes per-chunk partials that a
// per-row (or per-strip) kernel folds in chunk order, and the per-element
// vector kernels loop over the columns instead of holding them in registers.
// Every sum runs in a fixed order, so runs are bitwise reproducible.
#pragma once

#include <cfloat>
#include <cstdint>

#include "row.cuh"
#include "tile.cuh"

namespace dot_amd {
namespace spf {

constexpr int kColsPerThread = (kMaxRowLen + kBlock - 1) / kBlock;  // 16

struct Args {
    const float* X;  // log_alpha [B,M,N]
    float inv_tau;
    int B, M, N, rows, nstrips;
    float* lse;      // [B,M]
    float* u;        // [B,M]
    float* upart;    // [B,nstrips] strip sums of u
    float* v;        // [B,N]
    float* vpart;    // [B,nstrips,N]
    float* tau_est;  // [B]
    // rows longer than kMaxRowLen
    int nchunks;
    float2* rpart;   // [B,nchunks,M] chunk (max, sum) of the row log-sum-exp
    float* dpart;    // [B,nchunks,M] chunk sums of P v
};

// Centre this block's vector (kColsPerThread values per thread, columns
// threadIdx.x + q * kBlock < n) and divide it by its norm, as
// center_and_normalize (kernels.cu:71-126): mean = sum / n, then
// norm = sqrt(max(sum of squares, 1e-12)).
__device__ __forceinline__ void centre_normalise(float (&x)[kColsPerThread], int n, float* scratch) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < kColsPerThread; ++q)
        if (threadIdx.x + q * kBlock < n) s += x[q];
    const float mean = block_reduce<kWavesPerBlock>(wave_sum(s), scratch, OpSum{}) / static_cast<float>(n);
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < kColsPerThread; ++q)
        if (threadIdx.x + q * kBlock < n) {
            x[q] -= mean;
            ss += x[q] * x[q];
        }
    const float norm = sqrtf(fmaxf(block_reduce<kWavesPerBlock>(wave_sum(ss), scratch, OpSum{}), 1.0e-12f));
#pragma unroll
    for (int q = 0; q < kColsPerThread; ++q) x[q] /= norm;
}

// Row log-sum-exp: max_j of log_alpha * inv_tau, then
// max + log(max(sum safe_exp(. - max), 1e-12)) (kernels.cu:161-183).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void spf_lse(Args a) {
    using R = Row<VEC, CH>;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = blockIdx.x * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N, lane, a.N, x, 0.0f);
        float mx = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] *= a.inv_tau;
            if (R::valid(lane, e, a.N)) mx = fmaxf(mx, x[e]);
        }
        const float m = wave_max(mx);
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, a.N)) s += safe_exp(x[e] - m);
        s = wave_sum(s);
        if (lane == 0) a.lse[size_t(b) * a.M + i] = m + logf(fmaxf(s, 1.0e-12f));
    }
}

// v0 (kernels.cu:186-193), one block per batch element.
static __global__ __launch_bounds__(kBlock) void spf_init(Args a) {
    // the reference's float roundings of both products and of the sum, not a
    // contracted fma
#pragma clang fp contract(off)
    __shared__ float scratch[kWavesPerBlock];
    const int b = blockIdx.x;
    float x[kColsPerThread];
#pragma unroll
    for (int q = 0; q < kColsPerThread; ++q) {
        const int j = threadIdx.x + q * kBlock;
        const float t1 = static_cast<float>(j + 1) * 12.9898f;
        const float t2 = static_cast<float>(b + 1) * 78.233f;
        x[q] = j < a.N ? sinf(t1 + t2) : 0.0f;
    }
    centre_normalise(x, a.N, scratch);
#pragma unroll
    for (int q = 0; q < kColsPerThread; ++q) {
        const int j = threadIdx.x + q * kBlock;
        if (j < a.N) a.v[size_t(b) * a.N + j] = x[q];
    }
}

// u_i = sum_j P_ij v_j with P_ij = safe_exp(log_alpha_ij * inv_tau - lse_i)
// (kernels.cu:196-206), and this strip's sum of u.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void spf_rowdot(Args a) {
    using R = Row<VEC, CH>;
    __shared__ float scratch[kWavesPerBlock];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int st = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = st * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    float v[R::PL];
    R::load(a.v + size_t(b) * a.N, lane, a.N, v, 0.0f);
    float usum = 0.0f;  // lane 0: this wave's rows
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N, lane, a.N, x, 0.0f);
        const float lse = a.lse[size_t(b) * a.M + i];
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, a.N)) d = fmaf(safe_exp(x[e] * a.inv_tau - lse), v[e], d);
        d = wave_sum(d);
        if (lane == 0) {
            a.u[size_t(b) * a.M + i] = d;
            usum += d;
        }
    }
    const float s = block_reduce<kWavesPerBlock>(lane == 0 ? usum : 0.0f, scratch, OpSum{});
    if (threadIdx.x == 0) a.upart[size_t(b) * a.nstrips + st] = s;
}

// Mean of u over the element's rows from the strip sums, in strip order.
__device__ __forceinline__ float u_mean(const Args& a, int b) {
    float s = 0.0f;
    for (int k = 0; k < a.nstrips; ++k) s += a.upart[size_t(b) * a.nstrips + k];
    return s / static_cast<float>(a.M);
}

// Column partials of P_ij (u_i - mean u) over the strip (kernels.cu:208-218).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void spf_coldot(Args a) {
    using R = Row<VEC, CH>;
    extern __shared__ __align__(16) float lds[];  // block_column_combine: 2 N floats
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int st = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = st * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const float mean = u_mean(a, b);
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N, lane, a.N, x, 0.0f);
        const float lse = a.lse[size_t(b) * a.M + i];
        const float w = a.u[size_t(b) * a.M + i] - mean;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, a.N)) acc[e] = fmaf(safe_exp(x[e] * a.inv_tau - lse), w, acc[e]);
    }
    block_column_combine<VEC, CH>(acc, lds, a.N);
    if (wave == 0) R::store(a.vpart + (size_t(b) * a.nstrips + st) * a.N, lane, a.N, acc);
}

// v = sum of the strips' column partials (strip order), centred and normalised.
static __global__ __launch_bounds__(kBlock) void spf_vfold(Args a) {
    __shared__ float scratch[kWavesPerBlock];
    const int b = blockIdx.x;
    float x[kColsPerThread];
#pragma unroll
    for (int q = 0; q < kColsPerThread; ++q) {
        const int j = threadIdx.x + q * kBlock;
        float s = 0.0f;
        if (j < a.N)
            for (int k = 0; k < a.nstrips; ++k) s += a.vpart[(size_t(b) * a.nstrips + k) * a.N + j];
        x[q] = s;
    }
    centre_normalise(x, a.N, scratch);
#pragma unroll
    for (int q = 0; q < kColsPerThread; ++q) {
        const int j = threadIdx.x + q * kBlock;
        if (j < a.N) a.v[size_t(b) * a.N + j] = x[q];
    }
}

// tau_est = ||u - mean u|| = sqrt(max(sum, 1e-12)), clamped to [0, 0.999999]
// (kernels.cu:222-240).
static __global__ __launch_bounds__(kBlock) void spf_final(Args a) {
    __shared__ float scratch[kWavesPerBlock];
    const int b = blockIdx.x;
    const float mean = u_mean(a, b);
    float ss = 0.0f;
    for (int i = threadIdx.x; i < a.M; i += kBlock) {
        const float d = a.u[size_t(b) * a.M + i] - mean;
        ss += d * d;
    }
    const float norm = sqrtf(fmaxf(block_reduce<kWavesPerBlock>(wave_sum(ss), scratch, OpSum{}), 1.0e-12f));
    if (threadIdx.x == 0) a.tau_est[b] = fmaxf(0.0f, fminf(norm, 0.999999f));
}

// ---------------------------------------------------------------------------
// Rows longer than kMaxRowLen (nchunks > 1): strips x chunks tiles.
// ---------------------------------------------------------------------------

// Chunk partials of the row log-sum-exp: (max, sum safe_exp(. - max)).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void spf_lse_tiles(Args a) {
    using R = Row<VEC, CH>;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const wide::Tile tl = wide::tile_of_block(a.nchunks, a.N);
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N + tl.c0, lane, tl.nc, x, 0.0f);
        float mx = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] *= a.inv_tau;
            if (R::valid(lane, e, tl.nc)) mx = fmaxf(mx, x[e]);
        }
        const float m = wave_max(mx);
        float sm = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, tl.nc)) sm += safe_exp(x[e] - m);
        sm = wave_sum(sm);
        if (lane == 0) a.rpart[(size_t(b) * a.nchunks + tl.c) * a.M + i] = make_float2(m, sm);
    }
}

// lse_i from the chunk partials, one wave per row.
static __global__ __launch_bounds__(kBlock) void spf_lse_fold(Args a) {
    const int lane = threadIdx.x % kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int i = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (i >= a.M) return;
    float m, sm;
    wide::fold_lse(a.rpart + size_t(b) * a.nchunks * a.M + i, a.M, a.nchunks, m, sm);
    if (lane == 0) a.lse[size_t(b) * a.M + i] = m + logf(fmaxf(sm, 1.0e-12f));
}

// Chunk partials of u_i = sum_j P_ij v_j.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void spf_rowdot_tiles(Args a) {
    using R = Row<VEC, CH>;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const wide::Tile tl = wide::tile_of_block(a.nchunks, a.N);
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    float v[R::PL];
    R::load(a.v + size_t(b) * a.N + tl.c0, lane, tl.nc, v, 0.0f);
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N + tl.c0, lane, tl.nc, x, 0.0f);
        const float lse = a.lse[size_t(b) * a.M + i];
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, tl.nc)) d = fmaf(safe_exp(x[e] * a.inv_tau - lse), v[e], d);
        d = wave_sum(d);
        if (lane == 0) a.dpart[(size_t(b) * a.nchunks + tl.c) * a.M + i] = d;
    }
}

// u_i folded over the chunks (chunk order), and this strip's sum of u as
// spf_rowdot forms it; one workgroup per strip.
static __global__ __launch_bounds__(kBlock) void spf_rowdot_fold(Args a) {
    __shared__ float scratch[kWavesPerBlock];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int st = blockIdx.x;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const int r0 = st * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    float usum = 0.0f;  // lane 0: this wave's rows
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const float d = wide::fold_sum(a.dpart + size_t(b) * a.nchunks * a.M + i, a.M, a.nchunks);
        if (lane == 0) {
            a.u[size_t(b) * a.M + i] = d;
            usum += d;
        }
    }
    const float s = block_reduce<kWavesPerBlock>(lane == 0 ? usum : 0.0f, scratch, OpSum{});
    if (threadIdx.x == 0) a.upart[size_t(b) * a.nstrips + st] = s;
}

// Column partials of P_ij (u_i - mean u) over the tile's rows (the chunk's
// columns of the strip's partial row).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void spf_coldot_tiles(Args a) {
    using R = Row<VEC, CH>;
    extern __shared__ __align__(16) float lds[];  // block_column_combine: 2 kChunk floats
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int b = batch_of_block();
    if (b >= a.B) return;
    const wide::Tile tl = wide::tile_of_block(a.nchunks, a.N);
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const float mean = u_mean(a, b);
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (size_t(b) * a.M + i) * a.N + tl.c0, lane, tl.nc, x, 0.0f);
        const float lse = a.lse[size_t(b) * a.M + i];
        const float w = a.u[size_t(b) * a.M + i] - mean;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, tl.nc)) acc[e] = fmaf(safe_exp(x[e] * a.inv_tau - lse), w, acc[e]);
    }
    block_column_combine<VEC, CH>(acc, lds, tl.nc);
    if (wave == 0) R::store(a.vpart + (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0, lane, tl.nc, acc);
}

// centre_normalise for a vector of any length kept in global memory (this
// block's element only): thread t takes columns t, t + kBlock, ... in order,
// as the register version, re-reading what it wrote itself.
__device__ __forceinline__ void centre_normalise_mem(float* x, int n, float* scratch) {
    float s = 0.0f;
    for (int j = threadIdx.x; j < n; j += kBlock) s += x[j];
    const float mean = block_reduce<kWavesPerBlock>(wave_sum(s), scratch, OpSum{}) / static_cast<float>(n);
    float ss = 0.0f;
    for (int j = threadIdx.x; j < n; j += kBlock) {
        const float d = x[j] - mean;
        x[j] = d;
        ss += d * d;
    }
    const float norm = sqrtf(fmaxf(block_reduce<kWavesPerBlock>(wave_sum(ss), scratch, OpSum{}), 1.0e-12f));
    for (int j = threadIdx.x; j < n; j += kBlock) x[j] /= norm;
}

// spf_init for rows longer than kMaxRowLen.
static __global__ __launch_bounds__(kBlock) void spf_init_long(Args a) {
#pragma clang fp contract(off)
    __shared__ float scratch[kWavesPerBlock];
    const int b = blockIdx.x;
    float* v = a.v + size_t(b) * a.N;
    const float t2 = static_cast<float>(b + 1) * 78.233f;
    for (int j = threadIdx.x; j < a.N; j += kBlock) v[j] = sinf(static_cast<float>(j + 1) * 12.9898f + t2);
    centre_normalise_mem(v, a.N, scratch);
}

// spf_vfold for rows longer than kMaxRowLen.
static __global__ __launch_bounds__(kBlock) void spf_vfold_long(Args a) {
    __shared__ float scratch[kWavesPerBlock];
    const int b = blockIdx.x;
    float* v = a.v + size_t(b) * a.N;
    for (int j = threadIdx.x; j < a.N; j += kBlock) {
        float s = 0.0f;
        for (int k = 0; k < a.nstrips; ++k) s += a.vpart[(size_t(b) * a.nstrips + k) * a.N + j];
        v[j] = s;
    }
    centre_normalise_mem(v, a.N, scratch);
}

}  // namespace spf
}  // namespace dot_amd
