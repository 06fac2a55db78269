// Sinkhorn sweeps for rows longer than a wave can hold in registers (N > 4096).
//
// The streaming sweeps (sinkhorn_kernels.cuh) keep a whole row in a wave's
// registers, so a row's reduction and the column sums it feeds happen in one
// pass.  Here a row is cut into column chunks of kChunk floats and the grid
// is tiled strips x chunks: workgroup (s, c) of batch element b owns rows
// [s*rows, (s+1)*rows) and columns [c*kChunk, (c+1)*kChunk).  A row
// reduction therefore takes two passes over the matrix per iteration:
//
//   rows pass:    each tile writes its chunk's partial of every row it owns
//                 (log-sum-exp as (max, sum), or a plain sum) to a
//                 [B, nchunks, M] plane;
//   columns pass: each tile folds the nchunks partials of its rows in a fixed
//                 order (the row's finished value: u_i, lambda_i, ...), then
//                 accumulates that row's contribution to its chunk's column
//                 sums and writes them as one partial row per strip, in the
//                 [B, nstrips, N] layout the existing column combines read.
//
// This is the reference's chunked row and column phases (kernels.cuh:36-44,
// kernels.cu:547-627, :673-753) with every access a coalesced row access (the
// reference's column phases walk columns with stride N).  Nothing is reduced
// with float atomics, so results are bitwise reproducible.
#pragma once

#include <cfloat>
#include <cstdint>

#include "sinkhorn_kernels.cuh"
#include "tile.cuh"

namespace dot_amd {
namespace wide {

using sk::kSumFloor;

// -------------------------------------------------------------------------
// Forward
// -------------------------------------------------------------------------
struct FwdArgs {
    const float* X;        // scores [B,M,N]
    float kscale;          // K = X * kscale
    const float* log_a;    // [B,M] or null
    float log_a_default;
    const float* v_old;    // [B,N]
    const float* u_old;    // [B,M]
    float* u_new;          // [B,M]
    float* u_hist;         // [B,M] slice of the history, or null
    float2* rpart;         // [B,nchunks,M] (max, sum) of (K + v) log2 e over each chunk, base 2
    float* partial;        // [B,nstrips,N]
    unsigned* delta_bits;  // [max_iter+1]
    int B, M, N, rows, nstrips, nchunks, t;
    float tol;
};

// Rows pass of iteration t: per row and chunk, m = max_j(K_ij + v_j) and
// s = sum_j exp(K_ij + v_j - m) over the chunk's columns (kernels.cu:547-581),
// in base 2 as the streaming sweep (y = (K + v) log2 e, s = sum 2^(y - m)).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void fwd_rows(FwdArgs a) {
    if (sk::stopped_before(a.delta_bits, a.t, a.tol)) return;
    const int b = batch_of_block();
    if (b >= a.B) return;
    using R = Row<VEC, CH>;
    const Tile tl = tile_of_block(a.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float v2[R::PL];
    R::load(a.v_old + size_t(b) * a.N + tl.c0, lane, tl.nc, v2, 0.0f);
#pragma unroll
    for (int e = 0; e < R::PL; ++e) v2[e] *= kLog2E;
    const float kscale2 = a.kscale * kLog2E;
    float2* part = a.rpart + (size_t(b) * a.nchunks + tl.c) * a.M;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (bM + i) * a.N + tl.c0, lane, tl.nc, x, 0.0f);
        float mloc = -FLT_MAX;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            x[e] = R::valid(lane, e, tl.nc) ? fmaf(x[e], kscale2, v2[e]) : -INFINITY;
            mloc = fmaxf(mloc, x[e]);
        }
        const float m = wave_max(mloc);
        float sloc = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) sloc += __builtin_amdgcn_exp2f(x[e] - m);
        const float s = wave_sum(sloc);
        if (lane == 0) part[i] = make_float2(m, s);
    }
}

// Columns pass of iteration t: u_i = log a_i - (m_i + log max(s_i, 1e-12))
// from the folded chunk partials (kernels.cu:583-627; base 2 as fwd_rows), and the column sums
// sum_i exp(K_ij + u_i + v_j) = sum_i exp(K_ij + v_j - m_i) exp(log a_i - log s_i)
// of the chunk's columns, one partial row per strip (read by sk::fwd_combine).
// Chunk 0's tiles write u and the stop test's |u_t - u_{t-1}|.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void fwd_cols(FwdArgs a) {
    if (sk::stopped_before(a.delta_bits, a.t, a.tol)) return;
    const int b = batch_of_block();
    if (b >= a.B) return;
    using R = Row<VEC, CH>;
    extern __shared__ float lds[];
    const Tile tl = tile_of_block(a.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float v2[R::PL];
    R::load(a.v_old + size_t(b) * a.N + tl.c0, lane, tl.nc, v2, 0.0f);
    const float kscale2 = a.kscale * kLog2E;
    const float2* part = a.rpart + size_t(b) * a.nchunks * a.M;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        v2[e] *= kLog2E;
        acc[e] = 0.0f;
    }
    float dmax = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float x[R::PL];
        R::load(a.X + (bM + i) * a.N + tl.c0, lane, tl.nc, x, 0.0f);
        float m, ssum;
        fold_lse2(part + i, a.M, a.nchunks, m, ssum);
        const float lga = a.log_a ? a.log_a[bM + i] : a.log_a_default;
        const float lg2 = __builtin_amdgcn_logf(fmaxf(ssum, kSumFloor));  // log2
        const float u = lga - kLn2 * (m + lg2);
        const float w = __builtin_amdgcn_exp2f(fmaf(lga, kLog2E, -lg2));  // a / s
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float y = R::valid(lane, e, tl.nc) ? fmaf(x[e], kscale2, v2[e]) : -INFINITY;
            acc[e] = fmaf(__builtin_amdgcn_exp2f(y - m), w, acc[e]);
        }
        if (tl.c == 0 && lane == 0) {
            a.u_new[bM + i] = u;
            if (a.u_hist) a.u_hist[bM + i] = u;
            if (a.tol > 0.0f) dmax = fmaxf(dmax, fabsf(u - a.u_old[bM + i]));
        }
    }
    block_column_combine<VEC, CH>(acc, lds, tl.nc);
    if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0, lane, tl.nc, acc);
    if (a.tol > 0.0f && tl.c == 0) {
        const float bm = block_reduce<kWavesPerBlock>(dmax, lds + 2 * kChunk, OpMax{});
        if (threadIdx.x == 0) atomicMax(a.delta_bits + a.t, __float_as_uint(bm));
    }
}

// P = safe_exp(K + u_i + v_j) (kernels.cu:755-775) and per-tile sums of P * C,
// as sk::materialize for one chunk of columns; cost_partial is [B, gridDim.x].
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void materialize(sk::MaterializeArgs a, int nchunks) {
    const int b = batch_of_block();
    if (b >= a.B) return;
    using R = Row<VEC, CH>;
    __shared__ float scratch[kWavesPerBlock];
    const Tile tl = tile_of_block(nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int par = (*a.iters_used) & 1;
    const float* u = a.ubuf + (size_t(par) * a.B + b) * a.M;
    const float* vsrc = a.vbuf + (size_t(par) * a.B + b) * a.N + tl.c0;
    float v[R::PL];
    R::load(vsrc, lane, tl.nc, v, 0.0f);
    if (a.v_out && tl.s == 0 && wave == 0) R::store(a.v_out + size_t(b) * a.N + tl.c0, lane, tl.nc, v);
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const float csign = a.scores_kind < 0 ? 1.0f : -1.0f;  // C = -log_alpha
    float cacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N + tl.c0;
        float x[R::PL];
        R::load(a.X + off, lane, tl.nc, x, 0.0f);
        const float ui = u[i];
        float p[R::PL];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float lp = (x[e] * a.kscale + ui) + v[e];
            p[e] = a.return_log ? lp : safe_exp(lp);
            if (a.cost_partial && R::valid(lane, e, tl.nc)) cacc = fmaf(p[e], csign * x[e], cacc);
        }
        if (a.plan) R::store(a.plan + off, lane, tl.nc, p);
        if (a.u_out && tl.c == 0 && lane == 0) a.u_out[bM + i] = ui;
    }
    if (a.cost_partial) {
        const float t = block_reduce<kWavesPerBlock>(wave_sum(cacc), scratch, OpSum{});
        if (threadIdx.x == 0) a.cost_partial[size_t(b) * gridDim.x + blockIdx.x] = t;
    }
}

// -------------------------------------------------------------------------
// Implicit adjoint
// -------------------------------------------------------------------------
struct ImpArgs {
    sk::ImpArgs s;     // r, rs, lam, c, cs, mu, partA/B ([B,nstrips,N]), grad, tau_partial, ...
    float2* rpart;     // [B,nchunks,M]: chunk sums of P G and P (prologue)
    float* dpart;      // [B,nchunks,M]: chunk sums of P mu (each sweep)
    int B, nchunks;
};

// Prologue: chunk partials of r_i = sum_k P G and rs_i = sum_k P, and the
// column partials of both (as sk::imp_prep); lambda = 0.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void imp_prep(ImpArgs w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const sk::ImpArgs& a = w.s;
    extern __shared__ float lds[];
    const Tile tl = tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float2* part = w.rpart + (size_t(b) * w.nchunks + tl.c) * a.M;
    float accA[R::PL], accB[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) accA[e] = accB[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N + tl.c0;
        float p[R::PL], x[R::PL], G[R::PL];
        R::load(a.P + off, lane, tl.nc, p, 0.0f);
        sk::load_upstream<VEC, CH>(a.g, b, off, lane, tl.nc, x, G);
        float lr = 0.0f, lrs = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float pg = R::valid(lane, e, tl.nc) ? p[e] * G[e] : 0.0f;
            lr += pg;
            lrs += p[e];
            accA[e] += pg;
            accB[e] += p[e];
        }
        const float rr = wave_sum(lr);
        const float rrs = wave_sum(lrs);
        if (lane == 0) {
            part[i] = make_float2(rr, rrs);
            if (tl.c == 0) a.lam[bM + i] = 0.0f;
        }
    }
    block_column_combine<VEC, CH>(accA, lds, tl.nc);
    if (wave == 0) R::store(a.partA + (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0, lane, tl.nc, accA);
    block_column_combine<VEC, CH>(accB, lds, tl.nc);
    if (wave == 0) R::store(a.partB + (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0, lane, tl.nc, accB);
}

// r_i, rs_i from the prologue's chunk partials; one wave per row.
static __global__ __launch_bounds__(kBlock) void imp_row_totals(ImpArgs w) {
    const size_t rows = size_t(w.B) * w.s.M;
    const size_t row = size_t(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
    if (row >= rows) return;
    const size_t b = row / w.s.M, i = row % w.s.M;
    const float2 t = fold_sum2(w.rpart + b * w.nchunks * w.s.M + i, w.s.M, w.nchunks);
    if (threadIdx.x % kWave == 0) {
        w.s.r[row] = t.x;
        w.s.rs[row] = t.y;
    }
}

// Sweep, rows pass: chunk partials of sum_k P_ik mu_k.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void imp_rows(ImpArgs w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const sk::ImpArgs& a = w.s;
    const Tile tl = tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float mu[R::PL];
    R::load(a.mu + size_t(b) * a.N + tl.c0, lane, tl.nc, mu, 0.0f);
    float* part = w.dpart + (size_t(b) * w.nchunks + tl.c) * a.M;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float p[R::PL];
        R::load(a.P + (bM + i) * a.N + tl.c0, lane, tl.nc, p, 0.0f);
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e) d = fmaf(p[e], mu[e], d);
        const float dot = wave_sum(d);
        if (lane == 0) part[i] = dot;
    }
}

// Sweep, columns pass: lambda_i = (r_i - sum_k P mu) / max(rs_i, 1e-12)
// (kernels.cu:965-1005) from the folded dot, then the column partials
// sum_i P_ik lambda_i of the mu update (read by sk::imp_mu_combine).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void imp_cols(ImpArgs w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const sk::ImpArgs& a = w.s;
    extern __shared__ float lds[];
    const Tile tl = tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const float* part = w.dpart + size_t(b) * w.nchunks * a.M;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float p[R::PL];
        R::load(a.P + (bM + i) * a.N + tl.c0, lane, tl.nc, p, 0.0f);
        const float dot = fold_sum(part + i, a.M, w.nchunks);
        const float lam = (a.r[bM + i] - dot) / fmaxf(a.rs[bM + i], kSumFloor);
#pragma unroll
        for (int e = 0; e < R::PL; ++e) acc[e] = fmaf(p[e], lam, acc[e]);
        if (tl.c == 0 && lane == 0) a.lam[bM + i] = lam;
    }
    block_column_combine<VEC, CH>(acc, lds, tl.nc);
    if (wave == 0) R::store(a.partA + (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0, lane, tl.nc, acc);
}

// grad = P (G - lambda_i - mu_k) / tau and per-tile sums of grad * log_alpha,
// as sk::imp_final for one chunk; tau_partial is [B, gridDim.x].
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void imp_final(ImpArgs w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const sk::ImpArgs& a = w.s;
    __shared__ float scratch[kWavesPerBlock];
    const Tile tl = tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const bool cost_kind = a.g.scores_kind < 0;
    const float gc = a.g.gC ? a.g.gC[b * a.g.gc_step] : 0.0f;
    float mu[R::PL];
    R::load(a.mu + size_t(b) * a.N + tl.c0, lane, tl.nc, mu, 0.0f);
    float tacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N + tl.c0;
        float p[R::PL], x[R::PL], G[R::PL];
        R::load(a.P + off, lane, tl.nc, p, 0.0f);
        sk::load_upstream<VEC, CH>(a.g, b, off, lane, tl.nc, x, G);
        const float lam = a.lam[bM + i];
        float o[R::PL];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float gl = (p[e] * ((G[e] - lam) - mu[e])) * a.inv_tau;
            const float la = cost_kind ? -x[e] : x[e];
            if (R::valid(lane, e, tl.nc)) tacc = fmaf(gl, la, tacc);
            o[e] = cost_kind ? gc * p[e] - gl : gl - gc * p[e];
        }
        R::store_stream(a.grad + off, lane, tl.nc, o);
    }
    const float t = block_reduce<kWavesPerBlock>(wave_sum(tacc), scratch, OpSum{});
    if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + blockIdx.x] = t;
}

// -------------------------------------------------------------------------
// Unrolled backward
// -------------------------------------------------------------------------
struct UnrArgs {
    sk::UnrArgs s;     // gamma, partial ([B,nstrips,N]), colsum, grad, tau_partial, ...
    float* tpart;      // [B,nchunks,M]: chunk sums of Gamma_Y
    int B, nchunks;
};

template <int VEC, int CH>
__device__ __forceinline__ void unr_epilogue(const sk::UnrArgs& a, int b, size_t off, int lane, int nc,
                                             const float (&gam)[VEC * CH], const float (&p)[VEC * CH],
                                             const float (&x)[VEC * CH], float& tacc) {
    using R = Row<VEC, CH>;
    const bool cost_kind = a.g.scores_kind < 0;
    const float gc = a.g.gC ? a.g.gC[b * a.g.gc_step] : 0.0f;
    float o[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        const float gl = gam[e] * a.inv_tau;                              // kernels.cu:926-936
        const float la = cost_kind ? -x[e] : x[e];
        if (R::valid(lane, e, nc)) tacc = fmaf(gam[e], la, tacc);          // kernels.cu:938-963
        o[e] = cost_kind ? gc * p[e] - gl : gl - gc * p[e];
    }
    R::store_stream(a.grad + off, lane, nc, o);
}

// Gamma = G * P (kernels.cu:844-854) and its column partials, as sk::unr_init
// for one chunk; with no recorded steps it writes the gradient.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void unr_init(UnrArgs w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const sk::UnrArgs& a = w.s;
    extern __shared__ float lds[];
    const Tile tl = tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    float tacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N + tl.c0;
        float p[R::PL], x[R::PL], G[R::PL];
        R::load(a.P + off, lane, tl.nc, p, 0.0f);
        sk::load_upstream<VEC, CH>(a.g, b, off, lane, tl.nc, x, G);
        float gam[R::PL];
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            gam[e] = G[e] * p[e];
            acc[e] += gam[e];
        }
        if (a.final_step) unr_epilogue<VEC, CH>(a, b, off, lane, tl.nc, gam, p, x, tacc);
        else R::store(a.gamma + off, lane, tl.nc, gam);
    }
    if (a.final_step) {
        const float t = block_reduce<kWavesPerBlock>(wave_sum(tacc), lds, OpSum{});
        if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + blockIdx.x] = t;
    } else {
        block_column_combine<VEC, CH>(acc, lds, tl.nc);
        if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0, lane, tl.nc, acc);
    }
}

// Gamma_Y = Gamma - safe_exp(K + u_t + v_t) * colsum(Gamma) for one chunk of a row.
template <int VEC, int CH>
__device__ __forceinline__ void unr_column_part(const sk::UnrArgs& a, size_t off, size_t bN, int c0, int nc,
                                                float ui, int lane, float (&gam)[VEC * CH],
                                                float (&x)[VEC * CH]) {
    using R = Row<VEC, CH>;
    float vec[R::PL], cs[R::PL];
    R::load(a.gamma + off, lane, nc, gam, 0.0f);
    R::load(a.g.X + off, lane, nc, x, 0.0f);
    R::load(a.v_t + bN + c0, lane, nc, vec, 0.0f);
    R::load(a.colsum + bN + c0, lane, nc, cs, 0.0f);
#pragma unroll
    for (int e = 0; e < R::PL; ++e) {
        const float q = safe_fast_exp((x[e] * a.kscale + ui) + vec[e]);
        gam[e] = gam[e] - q * cs[e];
    }
}

// Step t, rows pass: chunk partials of rowsum(Gamma_Y).
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void unr_rows(UnrArgs w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const sk::UnrArgs& a = w.s;
    const Tile tl = tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const size_t bN = size_t(b) * a.N;
    float* part = w.tpart + (size_t(b) * w.nchunks + tl.c) * a.M;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        float gam[R::PL], x[R::PL];
        unr_column_part<VEC, CH>(a, (bM + i) * a.N + tl.c0, bN, tl.c0, tl.nc, a.u_t[bM + i], lane, gam, x);
        float tl_ = 0.0f;
#pragma unroll
        for (int e = 0; e < R::PL; ++e)
            if (R::valid(lane, e, tl.nc)) tl_ += gam[e];
        const float t = wave_sum(tl_);
        if (lane == 0) part[i] = t;
    }
}

// Step t, columns pass (kernels.cu:1660-1670):
//   Gamma = Gamma_Y - safe_exp(K + u_t + v_{t-1}) * rowsum(Gamma_Y),
// stored (or the gradient on the final step) with Gamma's column partials.
template <int VEC, int CH>
__global__ __launch_bounds__(kBlock) void unr_cols(UnrArgs w) {
    const int b = batch_of_block();
    if (b >= w.B) return;
    using R = Row<VEC, CH>;
    const sk::UnrArgs& a = w.s;
    extern __shared__ float lds[];
    const Tile tl = tile_of_block(w.nchunks, a.N);
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r0 = tl.s * a.rows;
    const int r1 = min(r0 + a.rows, a.M);
    const size_t bM = size_t(b) * a.M;
    const size_t bN = size_t(b) * a.N;
    const float* part = w.tpart + size_t(b) * w.nchunks * a.M;
    float acc[R::PL];
#pragma unroll
    for (int e = 0; e < R::PL; ++e) acc[e] = 0.0f;
    float tacc = 0.0f;
    for (int i = r0 + wave; i < r1; i += kWavesPerBlock) {
        const size_t off = (bM + i) * a.N + tl.c0;
        const float ui = a.u_t[bM + i];
        float gam[R::PL], x[R::PL];
        unr_column_part<VEC, CH>(a, off, bN, tl.c0, tl.nc, ui, lane, gam, x);
        const float ti = fold_sum(part + i, a.M, w.nchunks);
        float vec[R::PL];
        if (a.v_tm1) R::load(a.v_tm1 + bN + tl.c0, lane, tl.nc, vec, 0.0f);
#pragma unroll
        for (int e = 0; e < R::PL; ++e) {
            const float pe = safe_fast_exp((x[e] * a.kscale + ui) + (a.v_tm1 ? vec[e] : 0.0f));
            gam[e] = gam[e] - pe * ti;
            acc[e] += gam[e];
        }
        if (a.final_step) {
            float p[R::PL];
            R::load(a.P + off, lane, tl.nc, p, 0.0f);
            unr_epilogue<VEC, CH>(a, b, off, lane, tl.nc, gam, p, x, tacc);
        } else {
            R::store(a.gamma + off, lane, tl.nc, gam);
        }
    }
    if (a.final_step) {
        const float t = block_reduce<kWavesPerBlock>(wave_sum(tacc), lds, OpSum{});
        if (threadIdx.x == 0) a.tau_partial[size_t(b) * gridDim.x + blockIdx.x] = t;
    } else {
        block_column_combine<VEC, CH>(acc, lds, tl.nc);
        if (wave == 0) R::store(a.partial + (size_t(b) * a.nstrips + tl.s) * a.N + tl.c0, lane, tl.nc, acc);
    }
}

}  // namespace wide
}  // namespace dot_amd
