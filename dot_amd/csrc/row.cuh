// Row-in-registers layout shared by every sweep kernel.
//
// A wave owns whole rows.  Lane `l` holds, for chunk k = 0..CH-1, the VEC
// consecutive columns starting at k*64*VEC + l*VEC, so each chunk is one
// coalesced 64*VEC*4-byte access per wave (a 1 KiB float4 access when VEC=4).
// A row of up to 64*VEC*CH columns lives in VEC*CH registers per lane, which is
// what lets a sweep reduce a row across the wave and keep per-column partial
// sums in the same registers for all the rows the wave visits.
#pragma once

#include <hip/hip_runtime.h>
#include <cfloat>
#include <type_traits>

#include "wave.cuh"

namespace dot_amd {

constexpr int kBlock = 256;                 // threads per workgroup (4 waves)
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kMaxRowLen = 4096;            // longest row held in registers

// Batch-indexed grids: grid y holds at most 65535 batch elements, so larger
// batches spill into grid z.  batch_grid(x, B) launches x workgroups per
// element; a kernel takes its element from batch_of_block() and returns when
// it is >= B (the last z slab may be partly empty).
inline dim3 batch_grid(unsigned x, int B) {
    const int z = (B + 65534) / 65535;
    const int y = (B + z - 1) / z;
    return dim3(x, unsigned(y > 0 ? y : 1), unsigned(z > 0 ? z : 1));
}

__device__ __forceinline__ int batch_of_block() {
    return int(blockIdx.z) * int(gridDim.y) + int(blockIdx.y);
}

template <int VEC, int CH>
struct Row {
    static constexpr int PL = VEC * CH;  // floats per lane

    __device__ static __forceinline__ int col(int lane, int k) { return k * (kWave * VEC) + lane * VEC; }

    // Load a row; lanes past N receive `fill`.  VEC=4 requires N % 4 == 0 and a
    // 16-byte aligned row start.
    __device__ static __forceinline__ void load(const float* __restrict__ row, int lane, int N,
                                                float (&x)[PL], float fill) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int c = col(lane, k);
            if constexpr (VEC == 4) {
                if (c < N) {
                    const float4 t = *reinterpret_cast<const float4*>(row + c);
                    x[4 * k + 0] = t.x;
                    x[4 * k + 1] = t.y;
                    x[4 * k + 2] = t.z;
                    x[4 * k + 3] = t.w;
                } else {
                    x[4 * k + 0] = x[4 * k + 1] = x[4 * k + 2] = x[4 * k + 3] = fill;
                }
            } else {
                x[k] = (c < N) ? row[c] : fill;
            }
        }
    }

    // As load(), but lanes past N load the row's last element(s) (a cache hit)
    // instead of branching around the load.  With every load unconditional the
    // compiler's wait counts stay exact, so a row loaded ahead stays in flight
    // while earlier ones are used (pipelined_rows).
    __device__ static __forceinline__ void load_clamped(const float* __restrict__ row, int lane, int N,
                                                        float (&x)[PL], float fill) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int c = col(lane, k);
            const bool in = c < N;
            if constexpr (VEC == 4) {
                const float4 t = *reinterpret_cast<const float4*>(row + min(c, N - 4));
                x[4 * k + 0] = in ? t.x : fill;
                x[4 * k + 1] = in ? t.y : fill;
                x[4 * k + 2] = in ? t.z : fill;
                x[4 * k + 3] = in ? t.w : fill;
            } else {
                const float t = row[min(c, N - 1)];
                x[k] = in ? t : fill;
            }
        }
    }

    __device__ static __forceinline__ void store(float* __restrict__ row, int lane, int N,
                                                 const float (&x)[PL]) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int c = col(lane, k);
            if (c < N) {
                if constexpr (VEC == 4) {
                    *reinterpret_cast<float4*>(row + c) =
                        make_float4(x[4 * k + 0], x[4 * k + 1], x[4 * k + 2], x[4 * k + 3]);
                } else {
                    row[c] = x[k];
                }
            }
        }
    }

    // Store of a row that nothing reads back soon (outputs): non-temporal, so
    // the stream does not evict inputs that are read again from the caches.
    __device__ static __forceinline__ void store_stream(float* __restrict__ row, int lane, int N,
                                                        const float (&x)[PL]) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int c = col(lane, k);
            if (c < N) {
                if constexpr (VEC == 4) {
                    typedef float v4f __attribute__((ext_vector_type(4)));
                    const v4f v = {x[4 * k + 0], x[4 * k + 1], x[4 * k + 2], x[4 * k + 3]};
                    __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(row + c));
                } else {
                    __builtin_nontemporal_store(x[k], row + c);
                }
            }
        }
    }

    // This lane's VEC values of chunk k from an LDS (or any) array of N floats;
    // 0 past N.  VEC = 4 requires N % 4 == 0 and a 16-byte aligned array.
    __device__ static __forceinline__ void chunk(const float* v, int lane, int k, int N, float (&out)[VEC]) {
        const int c = col(lane, k);
        if constexpr (VEC == 4) {
            float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (c < N) t = *reinterpret_cast<const float4*>(v + c);
            out[0] = t.x;
            out[1] = t.y;
            out[2] = t.z;
            out[3] = t.w;
        } else {
            out[0] = c < N ? v[c] : 0.0f;
        }
    }

    // true when element e of this lane is a real column (< N)
    __device__ static __forceinline__ bool valid(int lane, int e, int N) {
        return col(lane, e / VEC) + (e % VEC) < N;
    }
};

// Sum the per-lane column accumulators of the 4 waves of a workgroup in a fixed
// order, ((w0 + w2) + (w1 + w3)), and leave the result in wave 0's `acc`.
// `lds` must hold 2*N floats.  Contains barriers: every thread must call it.
template <int VEC, int CH>
__device__ __forceinline__ void block_column_combine(float (&acc)[VEC * CH], float* lds, int N) {
    using R = Row<VEC, CH>;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if (wave >= 2) R::store(lds + (wave - 2) * N, lane, N, acc);
    __syncthreads();
    if (wave < 2) {
        float o[R::PL];
        R::load(lds + wave * N, lane, N, o, 0.0f);
#pragma unroll
        for (int e = 0; e < R::PL; ++e) acc[e] += o[e];
    }
    __syncthreads();
    if (wave == 1) R::store(lds, lane, N, acc);
    __syncthreads();
    if (wave == 0) {
        float o[R::PL];
        R::load(lds, lane, N, o, 0.0f);
#pragma unroll
        for (int e = 0; e < R::PL; ++e) acc[e] += o[e];
    }
}

// One row of a Row<VEC, CH> layout, as a value (row buffers of pipelined_rows).
template <class R>
struct RowBuf {
    float v[R::PL];
};

// Visits rows i0, i0 + step, ... (< r1) with each row's load issued one visit
// ahead, so it is in flight while the previous row is computed: load(i, buf)
// fills a Buf, body(i, buf) consumes it.  Two buffers alternate (unrolled by
// two, so no register copy has to wait for a load in flight); the look-ahead
// past the last row reloads that row, a cache hit, which keeps every load
// unconditional and the wait counts exact (load with Row::load_clamped).
template <class Buf, class Load, class Body>
__device__ __forceinline__ void pipelined_rows(int i0, int r1, int step, Load&& load, Body&& body) {
    if (i0 >= r1) return;
    Buf x, y;
    load(i0, x);
    for (int i = i0; i < r1; i += 2 * step) {
        load(min(i + step, r1 - 1), y);
        body(i, x);
        load(min(i + 2 * step, r1 - 1), x);
        if (i + step < r1) body(i + step, y);
    }
}

// Pick (VEC, CH) for a row length and call f(integral_constant<VEC>, integral_constant<CH>).
// Returns false when N is outside the register-resident range.
template <class F>
bool dispatch_row(int N, bool vec4, F&& f) {
    using std::integral_constant;
    if (N <= 0 || N > kMaxRowLen) return false;
    if (vec4) {
        const int chunks = (N + 255) / 256;
        if (chunks <= 1) f(integral_constant<int, 4>{}, integral_constant<int, 1>{});
        else if (chunks <= 2) f(integral_constant<int, 4>{}, integral_constant<int, 2>{});
        else if (chunks <= 4) f(integral_constant<int, 4>{}, integral_constant<int, 4>{});
        else if (chunks <= 8) f(integral_constant<int, 4>{}, integral_constant<int, 8>{});
        else f(integral_constant<int, 4>{}, integral_constant<int, 16>{});
    } else {
        const int chunks = (N + 63) / 64;
        if (chunks <= 1) f(integral_constant<int, 1>{}, integral_constant<int, 1>{});
        else if (chunks <= 2) f(integral_constant<int, 1>{}, integral_constant<int, 2>{});
        else if (chunks <= 4) f(integral_constant<int, 1>{}, integral_constant<int, 4>{});
        else if (chunks <= 8) f(integral_constant<int, 1>{}, integral_constant<int, 8>{});
        else if (chunks <= 16) f(integral_constant<int, 1>{}, integral_constant<int, 16>{});
        else if (chunks <= 32) f(integral_constant<int, 1>{}, integral_constant<int, 32>{});
        else f(integral_constant<int, 1>{}, integral_constant<int, 64>{});
    }
    return true;
}

}  // namespace dot_amd
