// Strips x chunks tiling of a [B, M, N] sweep for rows longer than a wave
// holds in registers: workgroup (s, c) of batch element b owns rows
// [s*rows, (s+1)*rows) and columns [c*kChunk, (c+1)*kChunk).  Row reductions
// become per-chunk partials, folded here in a fixed order.
#pragma once

#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "row.cuh"

namespace dot_amd {
namespace wide {

constexpr int kChunk = 2048;  // columns per tile: Row<4, 8> or Row<1, 32>, 32 floats per lane

inline int num_chunks(int N) { return (N + kChunk - 1) / kChunk; }

// Rows per strip: the largest power of two in [4, 64] that still gives the
// grid >= 1024 workgroups (4 per CU on 256 CUs) once multiplied by the chunks.
inline int strip_rows(int B, int M, int nchunks) {
    int r = 64;
    while (r > 4 && int64_t(B) * nchunks * ((M + r - 1) / r) < 1024) r /= 2;
    return r;
}

struct Tile {
    int s;   // strip
    int c;   // chunk
    int c0;  // first column of the chunk
    int nc;  // columns in the chunk
};

__device__ __forceinline__ Tile tile_of_block(int nchunks, int N) {
    Tile t;
    t.c = int(blockIdx.x) % nchunks;
    t.s = int(blockIdx.x) / nchunks;
    t.c0 = t.c * kChunk;
    t.nc = min(kChunk, N - t.c0);
    return t;
}

// Fold of row i's chunk partials (max, sum) of a log-sum-exp, stored with
// stride `stride` (chunk c at p[c * stride]): returns (m, s) with
// s = sum_c s_c exp(m_c - m), m = max_c m_c.  Lanes take chunks lane,
// lane + 64, ... (online merge), then the wave reduces; every lane gets the
// result.  Every lane of the wave must call it.
__device__ __forceinline__ void fold_lse(const float2* p, size_t stride, int nchunks, float& m, float& s) {
    const int lane = threadIdx.x % kWave;
    float lm = -FLT_MAX, ls = 0.0f;
    for (int c = lane; c < nchunks; c += kWave) {
        const float2 q = p[size_t(c) * stride];
        const float nm = fmaxf(lm, q.x);
        ls = ls * fast_exp(lm - nm) + q.y * fast_exp(q.x - nm);
        lm = nm;
    }
    m = wave_max(lm);
    s = wave_sum(ls * fast_exp(lm - m));
}

// fold_lse for partials in base 2: s = sum_c s_c 2^(m_c - m).
__device__ __forceinline__ void fold_lse2(const float2* p, size_t stride, int nchunks, float& m, float& s) {
    const int lane = threadIdx.x % kWave;
    float lm = -FLT_MAX, ls = 0.0f;
    for (int c = lane; c < nchunks; c += kWave) {
        const float2 q = p[size_t(c) * stride];
        const float nm = fmaxf(lm, q.x);
        ls = ls * __builtin_amdgcn_exp2f(lm - nm) + q.y * __builtin_amdgcn_exp2f(q.x - nm);
        lm = nm;
    }
    m = wave_max(lm);
    s = wave_sum(ls * __builtin_amdgcn_exp2f(lm - m));
}

// Plain sum of row i's chunk partials (same layout as fold_lse).
__device__ __forceinline__ float fold_sum(const float* p, size_t stride, int nchunks) {
    const int lane = threadIdx.x % kWave;
    float acc = 0.0f;
    for (int c = lane; c < nchunks; c += kWave) acc += p[size_t(c) * stride];
    return wave_sum(acc);
}

__device__ __forceinline__ float2 fold_sum2(const float2* p, size_t stride, int nchunks) {
    const int lane = threadIdx.x % kWave;
    float ax = 0.0f, ay = 0.0f;
    for (int c = lane; c < nchunks; c += kWave) {
        const float2 q = p[size_t(c) * stride];
        ax += q.x;
        ay += q.y;
    }
    return make_float2(wave_sum(ax), wave_sum(ay));
}

// Pick (VEC, CH) of a chunk tile: float4 columns when rows are 16-byte aligned.
template <class F>
void dispatch_chunk(bool vec4, F&& f) {
    using std::integral_constant;
    if (vec4) f(integral_constant<int, 4>{}, integral_constant<int, kChunk / 256>{});
    else f(integral_constant<int, 1>{}, integral_constant<int, kChunk / 64>{});
}

}  // namespace wide
}  // namespace dot_amd
