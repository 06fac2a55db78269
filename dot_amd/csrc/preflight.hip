// Spectral preflight C ABI: argument checks, workspace layout, launches.
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "host.hpp"
#include "preflight.cuh"

namespace dot_amd {
namespace {

struct SpfLayout {
    float *lse, *u, *upart, *v, *vpart;
    float2* rpart;  // rows longer than kMaxRowLen: [B,nchunks,M] chunk partials
    float* dpart;
    int rows, nstrips, nchunks;
    size_t bytes;
};

SpfLayout spf_layout(void* ws, int B, int M, int N) {
    Carver c(ws);
    SpfLayout L{};
    L.nchunks = N > kMaxRowLen ? wide::num_chunks(N) : 1;
    L.rows = L.nchunks > 1 ? wide::strip_rows(B, M, L.nchunks) : sweep_strip_rows(B, M);
    L.nstrips = M > 0 ? (M + L.rows - 1) / L.rows : 0;
    L.lse = c.take<float>(size_t(B) * M);
    L.u = c.take<float>(size_t(B) * M);
    L.upart = c.take<float>(size_t(B) * L.nstrips);
    L.v = c.take<float>(size_t(B) * N);
    L.vpart = c.take<float>(size_t(B) * L.nstrips * N);
    L.rpart = c.take<float2>(L.nchunks > 1 ? size_t(B) * L.nchunks * M : 0);
    L.dpart = c.take<float>(L.nchunks > 1 ? size_t(B) * L.nchunks * M : 0);
    L.bytes = c.used();
    return L;
}

}  // namespace
}  // namespace dot_amd

using namespace dot_amd;

extern "C" size_t dot_sinkhorn_spectral_preflight_workspace_bytes(int B, int M, int N) {
    if (B < 0 || M < 0 || N < 0) return 0;
    return spf_layout(nullptr, B, M, N).bytes;
}

extern "C" int dot_sinkhorn_spectral_preflight(const dot_spectral_preflight_args* a, dot_stream_t stream_) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (!a) return fail(DOT_ERR_INVALID_ARG, "args is NULL");
    const int B = a->B, M = a->M, N = a->N;
    if (B < 0 || M < 0 || N < 0) return fail(DOT_ERR_INVALID_ARG, "B, M and N must be >= 0");
    if (!(std::isfinite(a->tau) && a->tau > 0.0f)) return fail(DOT_ERR_INVALID_ARG, "tau must be > 0");
    if (a->n_power < 1) return fail(DOT_ERR_INVALID_ARG, "n_power must be >= 1");
    if (B == 0) return ok();
    if (!a->tau_est) return fail(DOT_ERR_INVALID_ARG, "tau_est is NULL");
    if (M == 0 || N == 0) return fail(DOT_ERR_INVALID_ARG, "M and N must be >= 1");
    if (!a->log_alpha) return fail(DOT_ERR_INVALID_ARG, "log_alpha is NULL");
    const SpfLayout L = spf_layout(a->workspace, B, M, N);
    if (!a->workspace || a->workspace_bytes < L.bytes)
        return fail(DOT_ERR_WORKSPACE, "workspace smaller than dot_sinkhorn_spectral_preflight_workspace_bytes()");
    spf::Args x{};
    x.X = a->log_alpha;
    x.inv_tau = 1.0f / a->tau;  // kernels.cu:1527
    x.B = B;
    x.M = M;
    x.N = N;
    x.rows = L.rows;
    x.nstrips = L.nstrips;
    x.lse = L.lse;
    x.u = L.u;
    x.upart = L.upart;
    x.v = L.v;
    x.vpart = L.vpart;
    x.tau_est = a->tau_est;
    x.nchunks = L.nchunks;
    x.rpart = L.rpart;
    x.dpart = L.dpart;
    const bool vec4 = (N % 4 == 0) && aligned16(a->log_alpha);
    const dim3 strips = batch_grid(unsigned(L.nstrips), B);
    if (L.nchunks > 1) {
        // rows longer than kMaxRowLen: strips x chunks tiles, partials folded per row
        const dim3 tiles = batch_grid(unsigned(L.nstrips * L.nchunks), B);
        const dim3 rowgrid = batch_grid(unsigned((M + kWavesPerBlock - 1) / kWavesPerBlock), B);
        const size_t tile_lds = size_t(2) * wide::kChunk * sizeof(float);
        wide::dispatch_chunk(vec4, [&](auto vc, auto cc) {
            constexpr int V = decltype(vc)::value;
            constexpr int C = decltype(cc)::value;
            ProfScope prof("spf", stream);
            hipLaunchKernelGGL((spf::spf_lse_tiles<V, C>), tiles, dim3(kBlock), 0, stream, x);
            hipLaunchKernelGGL(spf::spf_lse_fold, rowgrid, dim3(kBlock), 0, stream, x);
            hipLaunchKernelGGL(spf::spf_init_long, dim3(B), dim3(kBlock), 0, stream, x);
            for (int it = 0; it <= a->n_power; ++it) {
                hipLaunchKernelGGL((spf::spf_rowdot_tiles<V, C>), tiles, dim3(kBlock), 0, stream, x);
                hipLaunchKernelGGL(spf::spf_rowdot_fold, strips, dim3(kBlock), 0, stream, x);
                if (it == a->n_power) break;
                hipLaunchKernelGGL((spf::spf_coldot_tiles<V, C>), tiles, dim3(kBlock), tile_lds, stream, x);
                hipLaunchKernelGGL(spf::spf_vfold_long, dim3(B), dim3(kBlock), 0, stream, x);
            }
            hipLaunchKernelGGL(spf::spf_final, dim3(B), dim3(kBlock), 0, stream, x);
        });
        return check_launch("dot_sinkhorn_spectral_preflight");
    }
    const size_t comb_lds = (size_t(2) * N + 8) * sizeof(float);
    bool launched = dispatch_row(N, vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        ProfScope prof("spf", stream);
        hipLaunchKernelGGL((spf::spf_lse<V, C>), strips, dim3(kBlock), 0, stream, x);
        hipLaunchKernelGGL(spf::spf_init, dim3(B), dim3(kBlock), 0, stream, x);
        for (int it = 0; it < a->n_power; ++it) {
            hipLaunchKernelGGL((spf::spf_rowdot<V, C>), strips, dim3(kBlock), 0, stream, x);
            hipLaunchKernelGGL((spf::spf_coldot<V, C>), strips, dim3(kBlock), comb_lds, stream, x);
            hipLaunchKernelGGL(spf::spf_vfold, dim3(B), dim3(kBlock), 0, stream, x);
        }
        hipLaunchKernelGGL((spf::spf_rowdot<V, C>), strips, dim3(kBlock), 0, stream, x);
        hipLaunchKernelGGL(spf::spf_final, dim3(B), dim3(kBlock), 0, stream, x);
    });
    if (!launched) return fail(DOT_ERR_UNSUPPORTED, "row length outside the supported range");
    return check_launch("dot_sinkhorn_spectral_preflight");
}
