// Bidirectional-softmax C ABI: argument checks, workspace layout, launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>

#include "bidi_kernels.cuh"
#include "bidi_onepass.cuh"
#include "bidi_wide.cuh"
#include "coop.hpp"
#include "host.hpp"

namespace dot_amd {
namespace {

// Column chunks of a row: 1 when a row fits a wave's registers, else rows
// are swept in wide::kChunk-column tiles (bidi_wide.cuh).
int row_chunks(int L2) { return L2 > kMaxRowLen ? wide::num_chunks(L2) : 1; }

int strip_rows_bidi(int B, int L1, int nchunks) {
    static const int forced = [] {
        const char* s = std::getenv("DOT_AMD_ROWS");
        return s ? std::atoi(s) : 0;
    }();
    if (forced >= 1) return forced;
    int r = 64;
    while (r > 4 && int64_t(B) * nchunks * ((L1 + r - 1) / r) < 1024) r /= 2;
    return r;
}

size_t lds_bytes(int N) { return (size_t(2) * N + 8) * sizeof(float); }

// ---- one-pass tier (bidi_onepass.cuh)
namespace op = bidi::onepass;
static_assert(op::kMaxEpoch == DOT_BIDISOFTMAX_MAX_EPOCH, "epoch limit of the header");

// Groups of 32 workgroups: one per XCD (32 CUs each on gfx950), at most 8.
int onepass_groups() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cached[dev]) cached[dev] = std::max(1, std::min(op::kMaxGroups, device_cus() / op::kMembers)) + 1;
    return cached[dev] - 1;
}

// DOT_AMD_BIDI_ONEPASS=0 keeps every shape on the two-sweep kernels.
bool onepass_enabled() {
    const char* s = std::getenv("DOT_AMD_BIDI_ONEPASS");
    return !(s && *s == '0');
}

// Deadline of one exchange wait in s_memrealtime ticks (10 ns): 200 us, or
// DOT_AMD_BIDI_WAIT_TICKS (a negative value makes every workgroup take the
// fallback at once: a test of its bitwise agreement).
int onepass_wait_ticks() {
    const char* s = std::getenv("DOT_AMD_BIDI_WAIT_TICKS");
    return s && *s ? std::atoi(s) : 20000;
}

// Shapes of the one-pass tier: a batch element's rows fill one group (513..1024
// rows of 513..1024 columns), every group has an element, and the stage count
// fits the tag.
bool onepass_shape(int B, int L1, int L2) {
    const int G = onepass_groups();
    return onepass_enabled() && G > 0 && L1 > 512 && L1 <= op::kMaxRows && L2 > 512 && L2 <= op::kMaxCols &&
           L2 % 4 == 0 && B >= G && (B + G - 1) / G <= op::kMaxStages;
}

__global__ void zero_words(unsigned long long* p, size_t n) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        p[i] = 0ull;
}

// Exchange words of a one-pass launch: the caller's, or the workspace's
// cleared now (epoch 1).
bool onepass_exchange(void* caller, uint32_t epoch, unsigned long long* ws_words, hipStream_t stream,
                      op::Exchange& x) {
    if (caller) {
        if (epoch < 1 || epoch > op::kMaxEpoch) {
            fail(DOT_ERR_INVALID_ARG, "exchange_epoch must be in 1..DOT_BIDISOFTMAX_MAX_EPOCH");
            return false;
        }
        x.words = static_cast<unsigned long long*>(caller);
        x.epoch = epoch;
    } else {
        hipLaunchKernelGGL(zero_words, dim3(512), dim3(kBlock), 0, stream, ws_words, op::kExchangeWords);
        x.words = ws_words;
        x.epoch = 1;
    }
    x.groups = onepass_groups();
    x.wait_ticks = onepass_wait_ticks();
    x.local_ok = local_exchange_allowed();
    return true;
}

struct FwdLayout {
    float *part_m, *part_s, *row_stats, *col_stats;
    float2* rpart;  // rows longer than kMaxRowLen: [B, nchunks, L1] row partials
    unsigned long long* exchange;  // one-pass shapes: exchange words
    int rows, nstrips, nchunks;
    size_t bytes;
};

FwdLayout fwd_layout(void* ws, int B, int L1, int L2, bool own_stats) {
    Carver c(ws);
    FwdLayout L{};
    L.exchange = c.take<unsigned long long>(onepass_shape(B, L1, L2) ? op::kExchangeWords : 0);
    L.nchunks = row_chunks(L2);
    L.rows = strip_rows_bidi(B, L1, L.nchunks);
    L.nstrips = (L1 + L.rows - 1) / L.rows;
    L.part_m = c.take<float>(size_t(B) * L.nstrips * L2);
    L.part_s = c.take<float>(size_t(B) * L.nstrips * L2);
    L.rpart = c.take<float2>(L.nchunks > 1 ? size_t(B) * L.nchunks * L1 : 0);
    if (own_stats) {
        L.row_stats = c.take<float>(size_t(B) * 2 * L1);
        L.col_stats = c.take<float>(size_t(B) * 2 * L2);
    }
    L.bytes = c.used();
    return L;
}

struct BwdLayout {
    float *dot_r, *dot_c, *partial, *tau_partial;
    float* dpart;  // rows longer than kMaxRowLen: [B, nchunks, L1] row-dot partials
    unsigned long long* exchange;  // one-pass shapes: exchange words
    int rows, nstrips, nchunks;
    size_t bytes;
};

BwdLayout bwd_layout(void* ws, int B, int L1, int L2) {
    Carver c(ws);
    BwdLayout L{};
    L.exchange = c.take<unsigned long long>(onepass_shape(B, L1, L2) ? op::kExchangeWords : 0);
    L.nchunks = row_chunks(L2);
    L.rows = strip_rows_bidi(B, L1, L.nchunks);
    L.nstrips = (L1 + L.rows - 1) / L.rows;
    L.dot_r = c.take<float>(size_t(B) * L1);
    L.dot_c = c.take<float>(size_t(B) * L2);
    L.partial = c.take<float>(size_t(B) * L.nstrips * L2);
    L.tau_partial = c.take<float>(size_t(B) * L.nstrips * L.nchunks);
    L.dpart = c.take<float>(L.nchunks > 1 ? size_t(B) * L.nchunks * L1 : 0);
    L.bytes = c.used();
    return L;
}


__global__ void batch_sum(const float* partial, int nblk, float scale, float* out) {
    const int b = blockIdx.x;
    float s = 0.0f;
    for (int k = threadIdx.x; k < nblk; k += kWave) s += partial[size_t(b) * nblk + k];
    s = wave_sum(s);
    if (threadIdx.x == 0) out[b] = s * scale;
}

__global__ void fill_value(float* p, size_t n, float value) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += size_t(gridDim.x) * blockDim.x)
        p[i] = value;
}

int check_common(int B, int L1, int L2, float tau) {
    if (B < 0 || L1 < 0 || L2 < 0) return fail(DOT_ERR_INVALID_ARG, "B, L1 and L2 must be >= 0");
    if (!(std::isfinite(tau) && tau > 0.0f)) return fail(DOT_ERR_INVALID_ARG, "tau must be > 0");
    return DOT_OK;
}

}  // namespace
}  // namespace dot_amd

using namespace dot_amd;

extern "C" size_t dot_bidisoftmax_forward_workspace_bytes(int B, int L1, int L2) {
    if (B < 0 || L1 < 0 || L2 < 0) return 0;
    return fwd_layout(nullptr, B, L1, L2, true).bytes;
}

extern "C" int dot_bidisoftmax_forward(const dot_bidisoftmax_fwd_args* a, dot_stream_t stream_) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (!a) return fail(DOT_ERR_INVALID_ARG, "args is NULL");
    if (int rc = check_common(a->B, a->L1, a->L2, a->tau)) return rc;
    const int B = a->B, L1 = a->L1, L2 = a->L2;
    if (size_t(B) * L1 * L2 == 0) return ok();
    if (!a->sim || !a->out) return fail(DOT_ERR_INVALID_ARG, "sim and out must be non-NULL");
    const bool own_stats = !a->row_stats || !a->col_stats;
    const FwdLayout L = fwd_layout(a->workspace, B, L1, L2, own_stats);
    if (!a->workspace || a->workspace_bytes < L.bytes)
        return fail(DOT_ERR_WORKSPACE, "workspace smaller than dot_bidisoftmax_forward_workspace_bytes()");
    bidi::FwdArgs x{};
    x.sim = a->sim;
    x.lengths = a->lengths;
    x.inv_T = 1.0f / a->tau;  // kernels.cu:426
    x.B = B;
    x.L1 = L1;
    x.L2 = L2;
    x.rows = L.rows;
    x.nstrips = L.nstrips;
    x.row_stats = own_stats ? L.row_stats : a->row_stats;
    x.col_stats = own_stats ? L.col_stats : a->col_stats;
    x.part_m = L.part_m;
    x.part_s = L.part_s;
    x.out = a->out;
    x.row_sm = a->row_sm;
    x.col_sm = a->col_sm;
    const bool vec4 = (L2 % 4 == 0) && aligned16(a->sim) && aligned16(a->out) &&
                      (!a->row_sm || aligned16(a->row_sm)) && (!a->col_sm || aligned16(a->col_sm));
    if (vec4 && !a->row_sm && !a->col_sm && onepass_shape(B, L1, L2)) {
        op::FwdArgs1 o{};
        o.sim = a->sim;
        o.lengths = a->lengths;
        o.sc = x.inv_T * kLog2E;
        o.B = B;
        o.L1 = L1;
        o.L2 = L2;
        o.out = a->out;
        o.row_stats = x.row_stats;
        o.col_stats = x.col_stats;
        if (!onepass_exchange(a->exchange, a->exchange_epoch, L.exchange, stream, o.x)) return DOT_ERR_INVALID_ARG;
        const dim3 grid(unsigned(o.x.groups * op::kMembers));
        ProfScope prof("bidi_fwd_onepass", stream);
        // full tiles (no lengths, 1024 rows of 1024 or 768 columns): the bounds
        // are constants
        const bool tile = !a->lengths && L1 == op::kMaxRows;
        if (tile && L2 == 1024)
            hipLaunchKernelGGL((op::fwd_kernel<4, true>), grid, dim3(op::kThreads), 0, stream, o);
        else if (L2 > 768)
            hipLaunchKernelGGL((op::fwd_kernel<4, false>), grid, dim3(op::kThreads), 0, stream, o);
        else if (tile && L2 == 768)
            hipLaunchKernelGGL((op::fwd_kernel<3, true>), grid, dim3(op::kThreads), 0, stream, o);
        else
            hipLaunchKernelGGL((op::fwd_kernel<3, false>), grid, dim3(op::kThreads), 0, stream, o);
        return check_launch("dot_bidisoftmax_forward");
    }
    const dim3 strips = batch_grid(unsigned(L.nstrips), B);
    const dim3 fold_grid = batch_grid(unsigned((L2 + bidi::kFoldCols - 1) / bidi::kFoldCols), B);
    if (L.nchunks > 1) {
        bidi::wide_rows::Args w{};
        w.f = x;
        w.rpart = L.rpart;
        w.B = B;
        w.nchunks = L.nchunks;
        const dim3 tiles = batch_grid(unsigned(L.nstrips) * unsigned(L.nchunks), B);
        const unsigned row_blocks = unsigned((size_t(B) * L1 + kWavesPerBlock - 1) / kWavesPerBlock);
        wide::dispatch_chunk(vec4, [&](auto vc, auto cc) {
            constexpr int V = decltype(vc)::value;
            constexpr int C = decltype(cc)::value;
            {
                ProfScope prof("bidi_fwd_stats", stream);
                hipLaunchKernelGGL((bidi::wide_rows::fwd_stats<V, C>), tiles, dim3(kBlock),
                                   lds_bytes(wide::kChunk), stream, w);
            }
            {
                ProfScope prof("bidi_fwd_col_combine", stream);
                hipLaunchKernelGGL(bidi::wide_rows::fwd_row_stats, dim3(row_blocks), dim3(kBlock), 0, stream, w);
                hipLaunchKernelGGL(bidi::fwd_col_combine, fold_grid, dim3(kBlock), 0, stream, x);
            }
            {
                ProfScope prof("bidi_fwd_write", stream);
                hipLaunchKernelGGL((bidi::wide_rows::fwd_write<V, C>), tiles, dim3(kBlock),
                                   2 * size_t(wide::kChunk) * sizeof(float), stream, w);
            }
        });
        return check_launch("dot_bidisoftmax_forward");
    }
    bool launched = dispatch_row(L2, vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        {
            ProfScope prof("bidi_fwd_stats", stream);
            hipLaunchKernelGGL((bidi::fwd_stats<V, C>), strips, dim3(kBlock), lds_bytes(L2), stream, x);
        }
        {
            ProfScope prof("bidi_fwd_col_combine", stream);
            hipLaunchKernelGGL(bidi::fwd_col_combine, fold_grid, dim3(kBlock), 0, stream, x);
        }
        {
            ProfScope prof("bidi_fwd_write", stream);
            hipLaunchKernelGGL((bidi::fwd_write<V, C>), strips, dim3(kBlock),
                               (2 * size_t(L2) + 2 * L.rows) * sizeof(float), stream, x);
        }
    });
    if (!launched) return fail(DOT_ERR_UNSUPPORTED, "row length outside the supported range");
    return check_launch("dot_bidisoftmax_forward");
}

extern "C" size_t dot_bidisoftmax_exchange_bytes(void) { return op::kExchangeWords * sizeof(unsigned long long); }

extern "C" size_t dot_bidisoftmax_backward_workspace_bytes(int B, int L1, int L2) {
    if (B < 0 || L1 < 0 || L2 < 0) return 0;
    return bwd_layout(nullptr, B, L1, L2).bytes;
}

extern "C" int dot_bidisoftmax_backward(const dot_bidisoftmax_bwd_args* a, dot_stream_t stream_) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (!a) return fail(DOT_ERR_INVALID_ARG, "args is NULL");
    if (int rc = check_common(a->B, a->L1, a->L2, a->tau)) return rc;
    const int B = a->B, L1 = a->L1, L2 = a->L2;
    if (size_t(B) * L1 * L2 == 0) {
        if (B > 0 && a->grad_tau)
            hipLaunchKernelGGL(fill_value, dim3(1), dim3(kBlock), 0, stream, a->grad_tau, size_t(B), 0.0f);
        return check_launch("dot_bidisoftmax_backward");
    }
    if (!a->sim || !a->grad_out || !a->grad_sim)
        return fail(DOT_ERR_INVALID_ARG, "sim, grad_out and grad_sim must be non-NULL");
    const bool buffers = a->out && a->row_sm && a->col_sm;
    if (!buffers && !(a->row_stats && a->col_stats))
        return fail(DOT_ERR_INVALID_ARG,
                    "pass either (out, row_sm, col_sm) or (row_stats, col_stats)");
    const BwdLayout L = bwd_layout(a->workspace, B, L1, L2);
    if (!a->workspace || a->workspace_bytes < L.bytes)
        return fail(DOT_ERR_WORKSPACE, "workspace smaller than dot_bidisoftmax_backward_workspace_bytes()");
    bidi::BwdArgs x{};
    x.sim = a->sim;
    x.lengths = a->lengths;
    x.inv_T = 1.0f / a->tau;
    x.B = B;
    x.L1 = L1;
    x.L2 = L2;
    x.rows = L.rows;
    x.nstrips = L.nstrips;
    x.grad_out = a->grad_out;
    x.out = a->out;
    x.row_sm = a->row_sm;
    x.col_sm = a->col_sm;
    x.row_stats = a->row_stats;
    x.col_stats = a->col_stats;
    x.dot_r = L.dot_r;
    x.dot_c = L.dot_c;
    x.partial = L.partial;
    x.grad_sim = a->grad_sim;
    x.tau_partial = a->grad_tau ? L.tau_partial : nullptr;
    bool vec4 = (L2 % 4 == 0) && aligned16(a->sim) && aligned16(a->grad_out) && aligned16(a->grad_sim);
    if (!buffers && !a->grad_tau && vec4 && onepass_shape(B, L1, L2)) {
        op::BwdArgs1 o{};
        o.sim = a->sim;
        o.grad_out = a->grad_out;
        o.lengths = a->lengths;
        o.sc = x.inv_T * kLog2E;
        o.inv_T = x.inv_T;
        o.B = B;
        o.L1 = L1;
        o.L2 = L2;
        o.row_stats = a->row_stats;
        o.col_stats = a->col_stats;
        o.grad_sim = a->grad_sim;
        if (!onepass_exchange(a->exchange, a->exchange_epoch, L.exchange, stream, o.x)) return DOT_ERR_INVALID_ARG;
        const dim3 grid(unsigned(o.x.groups * op::kMembers));
        ProfScope prof("bidi_bwd_onepass", stream);
        // rows of exactly 1024 or 768 columns: the column bounds are constants
        if (L2 == 1024)
            hipLaunchKernelGGL((op::bwd_kernel<4, true>), grid, dim3(op::kThreads), 0, stream, o);
        else if (L2 > 768)
            hipLaunchKernelGGL((op::bwd_kernel<4, false>), grid, dim3(op::kThreads), 0, stream, o);
        else if (L2 == 768)
            hipLaunchKernelGGL((op::bwd_kernel<3, true>), grid, dim3(op::kThreads), 0, stream, o);
        else
            hipLaunchKernelGGL((op::bwd_kernel<3, false>), grid, dim3(op::kThreads), 0, stream, o);
        return check_launch("dot_bidisoftmax_backward");
    }
    if (buffers) vec4 = vec4 && aligned16(a->out) && aligned16(a->row_sm) && aligned16(a->col_sm);
    const dim3 strips = batch_grid(unsigned(L.nstrips), B);
    const dim3 fold_grid = batch_grid(unsigned((L2 + bidi::kFoldCols - 1) / bidi::kFoldCols), B);
    if (L.nchunks > 1) {
        bidi::wide_rows::Args w{};
        w.g = x;
        w.dpart = L.dpart;
        w.B = B;
        w.nchunks = L.nchunks;
        const dim3 tiles = batch_grid(unsigned(L.nstrips) * unsigned(L.nchunks), B);
        const unsigned row_blocks = unsigned((size_t(B) * L1 + kWavesPerBlock - 1) / kWavesPerBlock);
        wide::dispatch_chunk(vec4, [&](auto vc, auto cc) {
            constexpr int V = decltype(vc)::value;
            constexpr int C = decltype(cc)::value;
            auto run = [&](auto recompute) {
                constexpr bool RC = decltype(recompute)::value;
                {
                    ProfScope prof("bidi_bwd_dots", stream);
                    hipLaunchKernelGGL((bidi::wide_rows::bwd_dots<V, C, RC>), tiles, dim3(kBlock),
                                       2 * size_t(wide::kChunk) * sizeof(float) + lds_bytes(wide::kChunk),
                                       stream, w);
                }
                {
                    ProfScope prof("bidi_bwd_fold", stream);
                    hipLaunchKernelGGL(bidi::wide_rows::bwd_row_dots, dim3(row_blocks), dim3(kBlock), 0, stream, w);
                    hipLaunchKernelGGL(bidi::column_fold, fold_grid, dim3(kBlock), 0, stream, L.partial, L.nstrips,
                                       B, L2, L.dot_c);
                }
                {
                    ProfScope prof("bidi_bwd_write", stream);
                    hipLaunchKernelGGL((bidi::wide_rows::bwd_write<V, C, RC>), tiles, dim3(kBlock),
                                       3 * size_t(wide::kChunk) * sizeof(float), stream, w);
                }
            };
            if (buffers) run(std::false_type{});
            else run(std::true_type{});
        });
        if (a->grad_tau) {
            ProfScope prof("bidi_batch_sum", stream);
            hipLaunchKernelGGL(batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial, int(tiles.x), -x.inv_T,
                               a->grad_tau);
        }
        return check_launch("dot_bidisoftmax_backward");
    }
    bool launched = dispatch_row(L2, vec4, [&](auto vc, auto cc) {
        constexpr int V = decltype(vc)::value;
        constexpr int C = decltype(cc)::value;
        auto run = [&](auto recompute) {
            constexpr bool RC = decltype(recompute)::value;
            {
                ProfScope prof("bidi_bwd_dots", stream);
                hipLaunchKernelGGL((bidi::bwd_dots<V, C, RC>), strips, dim3(kBlock),
                                   (2 * size_t(L2) + 2 * L.rows) * sizeof(float) + lds_bytes(L2), stream, x);
            }
            {
                ProfScope prof("bidi_bwd_fold", stream);
                hipLaunchKernelGGL(bidi::column_fold, fold_grid, dim3(kBlock), 0, stream, L.partial, L.nstrips, B,
                                   L2, L.dot_c);
            }
            {
                ProfScope prof("bidi_bwd_write", stream);
                hipLaunchKernelGGL((bidi::bwd_write<V, C, RC>), strips, dim3(kBlock),
                                   (3 * size_t(L2) + 3 * L.rows) * sizeof(float), stream, x);
            }
        };
        if (buffers) run(std::false_type{});
        else run(std::true_type{});
        if (a->grad_tau) {
            ProfScope prof("bidi_batch_sum", stream);
            hipLaunchKernelGGL(batch_sum, dim3(B), dim3(kWave), 0, stream, L.tau_partial, L.nstrips,
                               -x.inv_T, a->grad_tau);
        }
    });
    if (!launched) return fail(DOT_ERR_UNSUPPORTED, "row length outside the supported range");
    return check_launch("dot_bidisoftmax_backward");
}
