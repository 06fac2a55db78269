// PyTorch binding of the dot_amd C ABI.
//
// * TORCH_LIBRARY(dot): the reference's eight schemas, verbatim
//   (src/sinkhorn/registry.cpp:31-56, src/bidirectional_softmax/registry.cpp:31-34),
//   so dot/_ops.py-style code binds the same torch.ops.dot.* handles.
// * TORCH_LIBRARY_IMPL(dot, CUDA): HIP tensors (PyTorch-ROCm dispatches them
//   under the CUDA key) go to the C ABI on the current HIP stream.
// * TORCH_LIBRARY(dot_amd): fused operators used by the Python autograd
//   functions (cost-fused forward, fused backward, statistics-based
//   bidirectional softmax).  HIP only.
//
// CPU tensors are served by cpu_ops.cpp.  No GPU tensor is ever computed on
// the CPU: a missing or failing HIP path raises.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/library.h>

#include <cmath>
#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/dot_amd.h"

namespace {

using at::Tensor;
using c10::optional;

void check_rc(int rc, const char* what) {
    TORCH_CHECK(rc == DOT_OK, what, " failed (code ", rc, "): ", dot_last_error());
}

dot_stream_t current_stream(const Tensor& t) {
    return reinterpret_cast<dot_stream_t>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_hip_input(const Tensor& t, const char* name) {
    TORCH_CHECK(t.device().is_cuda(), name, " must be a CUDA tensor");
}

Tensor f32c(const Tensor& t) { return t.to(at::kFloat).contiguous(); }

Tensor workspace(size_t bytes, const Tensor& like) {
    return at::empty({static_cast<int64_t>(std::max<size_t>(bytes, 1))},
                     like.options().dtype(at::kByte));
}

// Exchange words of the kernels whose workgroups exchange tagged words (the
// one-pass bidirectional softmax, the register-resident Sinkhorn tier), one
// set per operator and (device, stream): calls on one stream run in order, so
// no two kernels use a set at once, and the growing epoch keeps a call from
// reading words an earlier call left.  Cleared once (and again when the epoch
// would pass its limit); held until the process ends (the map is never
// destroyed, so no device memory is freed during interpreter teardown).
//
// Two cases get no set ({nullptr, 0}: the library then takes the words from
// the call's workspace and clears them with a kernel of the call):
//  * a stream under graph capture: the epoch is fixed when the call is
//    recorded, so every replay would poll for tags that the previous replay
//    already wrote; a clearing kernel recorded with the call runs on every
//    replay instead;
//  * a stream beyond the first kMaxSetsPerDevice of its device, so that
//    programs that cycle through many streams do not hold a set for each.
constexpr size_t kMaxSetsPerDevice = 16;

struct ExchangeSet {
    Tensor words;
    uint32_t epoch = 0;
};

bool stream_capturing(void* stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs) != hipSuccess ||
           cs != hipStreamCaptureStatusNone;
}

template <size_t (*Bytes)(), uint32_t MaxEpoch>
std::pair<void*, uint32_t> stream_exchange(const Tensor& like) {
    static std::mutex mu;
    static auto* sets = new std::map<std::pair<int, void*>, ExchangeSet>();
    static auto* per_device = new std::map<int, size_t>();
    const int dev = like.device().index();
    void* stream = c10::hip::getCurrentHIPStream(dev).stream();
    if (stream_capturing(stream)) return {nullptr, 0};
    std::lock_guard<std::mutex> lock(mu);
    auto it = sets->find({dev, stream});
    if (it == sets->end()) {
        if ((*per_device)[dev] >= kMaxSetsPerDevice) return {nullptr, 0};
        ++(*per_device)[dev];
        it = sets->emplace(std::make_pair(dev, stream), ExchangeSet{}).first;
    }
    ExchangeSet& x = it->second;
    if (!x.words.defined() || x.epoch >= MaxEpoch) {
        if (!x.words.defined())
            x.words = at::empty({static_cast<int64_t>(Bytes())}, like.options().dtype(at::kByte));
        x.words.zero_();  // on the current stream, ahead of the kernel
        x.epoch = 0;
    }
    return {x.words.data_ptr(), ++x.epoch};
}

std::pair<void*, uint32_t> bidi_exchange(const Tensor& like) {
    return stream_exchange<dot_bidisoftmax_exchange_bytes, DOT_BIDISOFTMAX_MAX_EPOCH>(like);
}

std::pair<void*, uint32_t> sinkhorn_exchange(const Tensor& like) {
    return stream_exchange<dot_sinkhorn_exchange_bytes, DOT_SINKHORN_MAX_EPOCH>(like);
}

const float* ptr_or_null(const optional<Tensor>& t) {
    return t.has_value() ? t->data_ptr<float>() : nullptr;
}

// Shape checks of torch_cuda.cpp:286-302.
void check_marginals(const optional<Tensor>& log_a, const optional<Tensor>& log_b, int64_t B,
                     int64_t n, int64_t m) {
    if (log_a.has_value()) {
        check_hip_input(*log_a, "*log_a");
        TORCH_CHECK(log_a->dim() == 2 && log_a->size(0) == B && log_a->size(1) == n,
                    "log_a must have shape [B, n]");
    }
    if (log_b.has_value()) {
        check_hip_input(*log_b, "*log_b");
        TORCH_CHECK(log_b->dim() == 2 && log_b->size(0) == B && log_b->size(1) == m,
                    "log_b must have shape [B, m]");
    }
}

struct ForwardOut {
    Tensor plan, cost, counts, u_hist, v_hist;
};

// One call of dot_sinkhorn_forward; counts = int32 [2] on the device: (iters_used, converged).
// counts_on_host: [iters_used, converged] go to pinned host memory, written
// there by the forward's last kernel (no device-to-host copy); valid once the
// stream has passed the call.
ForwardOut run_forward(const Tensor& scores_f, int kind, double tau, int64_t n_iters, double tol,
                       const optional<Tensor>& log_a_f, const optional<Tensor>& log_b_f,
                       bool return_log, bool want_plan, bool want_cost, bool keep_history,
                       bool counts_on_host = false) {
    const int64_t B = scores_f.size(0), M = scores_f.size(1), N = scores_f.size(2);
    TORCH_CHECK(n_iters <= INT32_MAX, "n_iters too large");
    auto opts = scores_f.options().dtype(at::kFloat);
    ForwardOut o;
    if (want_plan) o.plan = at::empty({B, M, N}, opts);
    if (want_cost) o.cost = at::empty({B}, opts);
    o.counts = counts_on_host ? at::empty({2}, at::TensorOptions().dtype(at::kInt).pinned_memory(true))
                              : at::empty({2}, scores_f.options().dtype(at::kInt));
    const int flags = (return_log ? DOT_SK_RETURN_LOG : 0) | (keep_history ? DOT_SK_KEEP_HISTORY : 0);
    if (keep_history) {
        o.u_hist = at::empty({n_iters, B, M}, opts);
        o.v_hist = at::empty({n_iters, B, N}, opts);
    }
    const size_t ws_bytes = dot_sinkhorn_forward_workspace_bytes(int(B), int(M), int(N), int(n_iters), flags);
    Tensor ws = workspace(ws_bytes, scores_f);
    dot_sinkhorn_fwd_args a{};
    a.scores = scores_f.data_ptr<float>();
    a.log_a = ptr_or_null(log_a_f);
    a.log_b = ptr_or_null(log_b_f);
    a.B = int(B);
    a.M = int(M);
    a.N = int(N);
    a.scores_kind = kind;
    a.tau = static_cast<float>(tau);
    a.max_iter = int(n_iters);
    a.tol = static_cast<float>(tol);
    a.flags = flags;
    a.plan = want_plan ? o.plan.data_ptr<float>() : nullptr;
    a.cost = want_cost ? o.cost.data_ptr<float>() : nullptr;
    a.u_hist = keep_history ? o.u_hist.data_ptr<float>() : nullptr;
    a.v_hist = keep_history ? o.v_hist.data_ptr<float>() : nullptr;
    a.iters_used = o.counts.data_ptr<int32_t>();
    a.converged = o.counts.data_ptr<int32_t>() + 1;
    a.workspace = ws.data_ptr();
    a.workspace_bytes = ws_bytes;
    std::tie(a.exchange, a.exchange_epoch) = sinkhorn_exchange(scores_f);
    check_rc(dot_sinkhorn_forward(&a, current_stream(scores_f)), "dot_sinkhorn_forward");
    return o;
}

optional<Tensor> f32c_opt(const optional<Tensor>& t) {
    if (!t.has_value()) return c10::nullopt;
    return f32c(*t);
}

void check_common(const Tensor& log_alpha, double tau, int64_t n_iters) {
    check_hip_input(log_alpha, "log_alpha");
    TORCH_CHECK(log_alpha.dim() == 3, "log_alpha must be 3D [B, n, m]");
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    TORCH_CHECK(n_iters >= 0, "n_iters must be >= 0");
}

// ---------------------------------------------------------------------------
// torch.ops.dot.* on HIP tensors
// ---------------------------------------------------------------------------

// sinkhorn / sinkhorn_log (torch_cuda.cpp:599-715).  The reference runs the
// primal full-matrix iteration here; the dual iteration with tol = 0 computes
// the same plan (test_sinkhorn.py:792-803 holds them to 1e-5).
Tensor sinkhorn_hip(const Tensor& log_alpha, double tau, int64_t n_iters,
                    const optional<Tensor>& log_a, const optional<Tensor>& log_b, bool return_log) {
    check_common(log_alpha, tau, n_iters);
    check_marginals(log_a, log_b, log_alpha.size(0), log_alpha.size(1), log_alpha.size(2));
    c10::OptionalDeviceGuard guard(log_alpha.device());
    return run_forward(f32c(log_alpha), DOT_SCORES_LOG_ALPHA, tau, n_iters, 0.0, f32c_opt(log_a),
                       f32c_opt(log_b), return_log, true, false, false)
        .plan;
}

Tensor sinkhorn_op(Tensor log_alpha, double tau, int64_t n_iters, optional<Tensor> log_a,
                   optional<Tensor> log_b) {
    return sinkhorn_hip(log_alpha, tau, n_iters, log_a, log_b, false);
}

Tensor sinkhorn_log_op(Tensor log_alpha, double tau, int64_t n_iters, optional<Tensor> log_a,
                       optional<Tensor> log_b) {
    return sinkhorn_hip(log_alpha, tau, n_iters, log_a, log_b, true);
}

std::vector<Tensor> counts_to_cpu(const Tensor& counts) {
    Tensor c = counts.to(at::kCPU);
    const int32_t* p = c.data_ptr<int32_t>();
    TORCH_CHECK(p[0] >= 0, "dot_sinkhorn_forward: a cross-workgroup exchange timed out (outputs are NaN)");
    auto opt = at::TensorOptions().dtype(at::kLong).device(at::kCPU);
    return {at::scalar_tensor(int64_t(p[0]), opt), at::scalar_tensor(int64_t(p[1]), opt)};
}

struct MethodParams {
    int64_t method = 0;
    double omega = 1.5;
    int64_t anderson_k = 5;
    double mixing_beta = 1.0, lr = 1.0, beta1 = 0.9, beta2 = 0.999, eps_adam = 1e-8;
    bool bias_correction = true;
    double reg_start = -1.0;
    int64_t schedule = 0;
};

// One call of dot_sinkhorn_forward_method (momentum / Anderson / Adam and the
// regularisation schedules); counts as for run_forward.
ForwardOut run_forward_method(const Tensor& scores_f, int kind, double tau, int64_t n_iters, double tol,
                              const optional<Tensor>& log_a_f, const optional<Tensor>& log_b_f,
                              bool return_log, bool want_cost, const MethodParams& mp) {
    const int64_t B = scores_f.size(0), M = scores_f.size(1), N = scores_f.size(2);
    TORCH_CHECK(n_iters <= INT32_MAX, "n_iters too large");
    TORCH_CHECK(mp.anderson_k <= INT32_MAX, "anderson_k too large");
    auto opts = scores_f.options().dtype(at::kFloat);
    ForwardOut o;
    o.plan = at::empty({B, M, N}, opts);
    if (want_cost) o.cost = at::empty({B}, opts);
    o.counts = at::empty({2}, scores_f.options().dtype(at::kInt));
    const int k = int(std::min<int64_t>(mp.anderson_k, INT32_MAX));
    const size_t ws_bytes = dot_sinkhorn_forward_method_workspace_bytes(int(B), int(M), int(N), int(n_iters),
                                                                        int(mp.method), k);
    Tensor ws = workspace(ws_bytes, scores_f);
    dot_sinkhorn_method_args m{};
    dot_sinkhorn_fwd_args& a = m.base;
    a.scores = scores_f.data_ptr<float>();
    a.log_a = ptr_or_null(log_a_f);
    a.log_b = ptr_or_null(log_b_f);
    a.B = int(B);
    a.M = int(M);
    a.N = int(N);
    a.scores_kind = kind;
    a.tau = static_cast<float>(tau);
    a.max_iter = int(n_iters);
    a.tol = static_cast<float>(tol);
    a.flags = return_log ? DOT_SK_RETURN_LOG : 0;
    a.plan = o.plan.data_ptr<float>();
    a.cost = want_cost ? o.cost.data_ptr<float>() : nullptr;
    a.iters_used = o.counts.data_ptr<int32_t>();
    a.converged = o.counts.data_ptr<int32_t>() + 1;
    a.workspace = ws.data_ptr();
    a.workspace_bytes = ws_bytes;
    std::tie(a.exchange, a.exchange_epoch) = sinkhorn_exchange(scores_f);
    m.method = int(mp.method);
    m.omega = static_cast<float>(mp.omega);
    m.anderson_k = int(std::min<int64_t>(mp.anderson_k, INT32_MAX));
    m.mixing_beta = static_cast<float>(mp.mixing_beta);
    m.lr = static_cast<float>(mp.lr);
    m.beta1 = static_cast<float>(mp.beta1);
    m.beta2 = static_cast<float>(mp.beta2);
    m.eps_adam = static_cast<float>(mp.eps_adam);
    m.bias_correction = mp.bias_correction ? 1 : 0;
    m.reg_start = static_cast<float>(mp.reg_start);
    m.schedule = int(mp.schedule);
    check_rc(dot_sinkhorn_forward_method(&m, current_stream(scores_f)), "dot_sinkhorn_forward_method");
    return o;
}

// sinkhorn_dual_forward (torch_cuda.cpp:266-557): returns [P or log P,
// used (CPU int64 0-d), converged (CPU int64 0-d)].  method 0 without a
// schedule is dot_sinkhorn_forward; the methods and schedules are
// dot_sinkhorn_forward_method.
std::vector<Tensor> sinkhorn_dual_forward_op(Tensor log_alpha, double tau, int64_t n_iters, double tol,
                                             optional<Tensor> log_a, optional<Tensor> log_b,
                                             bool return_log, int64_t method, double omega,
                                             int64_t anderson_k, double mixing_beta, double lr,
                                             double beta1, double beta2, double eps_adam,
                                             bool bias_correction, double reg_start, int64_t schedule) {
    check_common(log_alpha, tau, n_iters);
    TORCH_CHECK(anderson_k >= 1, "anderson_k must be >= 1");
    check_marginals(log_a, log_b, log_alpha.size(0), log_alpha.size(1), log_alpha.size(2));
    c10::OptionalDeviceGuard guard(log_alpha.device());
    ForwardOut o;
    if (method == 0 && schedule == 0) {
        o = run_forward(f32c(log_alpha), DOT_SCORES_LOG_ALPHA, tau, n_iters, tol, f32c_opt(log_a),
                        f32c_opt(log_b), return_log, true, false, false);
    } else {
        MethodParams mp{method, omega, anderson_k, mixing_beta, lr, beta1, beta2, eps_adam,
                        bias_correction, reg_start, schedule};
        o = run_forward_method(f32c(log_alpha), DOT_SCORES_LOG_ALPHA, tau, n_iters, tol, f32c_opt(log_a),
                               f32c_opt(log_b), return_log, false, mp);
    }
    std::vector<Tensor> c = counts_to_cpu(o.counts);
    return {o.plan, c[0], c[1]};
}

// sinkhorn_spectral_preflight (torch_cuda.cpp:559-593; kernel kernels.cu:141-241).
Tensor sinkhorn_spectral_preflight_op(Tensor log_alpha, double tau, int64_t n_power) {
    check_hip_input(log_alpha, "log_alpha");
    TORCH_CHECK(log_alpha.dim() == 3, "log_alpha must be 3D [B, n, m]");
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    TORCH_CHECK(n_power >= 1, "n_power must be >= 1");
    c10::OptionalDeviceGuard guard(log_alpha.device());
    Tensor X = f32c(log_alpha);
    const int64_t B = X.size(0), M = X.size(1), N = X.size(2);
    Tensor tau_est = at::empty({B}, X.options());
    const size_t ws_bytes = dot_sinkhorn_spectral_preflight_workspace_bytes(int(B), int(M), int(N));
    Tensor ws = workspace(ws_bytes, X);
    dot_spectral_preflight_args a{};
    a.log_alpha = X.data_ptr<float>();
    a.B = int(B);
    a.M = int(M);
    a.N = int(N);
    a.tau = static_cast<float>(tau);
    a.n_power = int(n_power);
    a.tau_est = tau_est.data_ptr<float>();
    a.workspace = ws.data_ptr();
    a.workspace_bytes = ws_bytes;
    check_rc(dot_sinkhorn_spectral_preflight(&a, current_stream(X)), "dot_sinkhorn_spectral_preflight");
    return tau_est;
}

// DOT_AMD_EXACT_SWEEPS=1: the implicit adjoint runs exactly backward_iters
// sweeps (DOT_SK_EXACT_SWEEPS) instead of ending each element once converged.
int backward_flags() {
    const char* e = std::getenv("DOT_AMD_EXACT_SWEEPS");
    return (e && e[0] == '1') ? DOT_SK_EXACT_SWEEPS : 0;
}

// status_on_host: the status word is pinned host memory that the backward's
// last kernel writes through, so reading it needs no device-to-host copy; it
// is followed there by the adjoint sweeps executed per batch element
// (implicit), which the adjoint kernel writes the same way.
// grad_cost_scalar: grad_cost holds one value that is every batch element's.
std::vector<Tensor> run_backward(bool implicit, const Tensor& scores_f, int kind, const Tensor& plan,
                                 const optional<Tensor>& grad_plan, const optional<Tensor>& grad_cost,
                                 double tau, int64_t iters, const Tensor& u_hist, const Tensor& v_hist,
                                 bool status_on_host = false, bool grad_cost_scalar = false) {
    const int64_t B = scores_f.size(0), M = scores_f.size(1), N = scores_f.size(2);
    auto opts = scores_f.options().dtype(at::kFloat);
    Tensor grad = at::empty({B, M, N}, opts);
    Tensor grad_tau = at::empty({B}, opts);
    const int64_t words = (status_on_host && implicit) ? 1 + B : 1;
    Tensor status = status_on_host ? at::empty({words}, at::TensorOptions().dtype(at::kInt).pinned_memory(true))
                                   : at::empty({1}, scores_f.options().dtype(at::kInt));
    const size_t ws_bytes = implicit ? dot_sinkhorn_backward_implicit_workspace_bytes(int(B), int(M), int(N))
                                     : dot_sinkhorn_backward_unrolled_workspace_bytes(int(B), int(M), int(N));
    Tensor ws = workspace(ws_bytes, scores_f);
    dot_sinkhorn_bwd_args a{};
    a.scores = scores_f.data_ptr<float>();
    a.scores_kind = kind;
    a.plan = plan.data_ptr<float>();
    a.grad_plan = ptr_or_null(grad_plan);
    a.grad_cost = ptr_or_null(grad_cost);
    a.B = int(B);
    a.M = int(M);
    a.N = int(N);
    a.tau = static_cast<float>(tau);
    TORCH_CHECK(iters <= INT32_MAX, "iteration count too large");
    a.iters = int(iters);
    a.u_hist = u_hist.defined() ? u_hist.data_ptr<float>() : nullptr;
    a.v_hist = v_hist.defined() ? v_hist.data_ptr<float>() : nullptr;
    a.grad_scores = grad.data_ptr<float>();
    a.grad_tau = grad_tau.data_ptr<float>();
    a.workspace = ws.data_ptr();
    a.workspace_bytes = ws_bytes;
    a.status = status.data_ptr<int32_t>();
    a.sweeps_used = words > 1 ? status.data_ptr<int32_t>() + 1 : nullptr;
    a.flags = (implicit ? backward_flags() : 0) | (grad_cost_scalar ? DOT_SK_GRAD_COST_SCALAR : 0);
    std::tie(a.exchange, a.exchange_epoch) = sinkhorn_exchange(scores_f);
    const dot_stream_t s = current_stream(scores_f);
    if (implicit) check_rc(dot_sinkhorn_backward_implicit(&a, s), "dot_sinkhorn_backward_implicit");
    else check_rc(dot_sinkhorn_backward_unrolled(&a, s), "dot_sinkhorn_backward_unrolled");
    return {grad, grad_tau, status};
}

// The reference's with_grads ops synchronise the device (cudaMalloc/cudaFree,
// torch_cuda.cpp:803-871), so these ops check here, with one copy, that no
// cross-workgroup exchange of the forward or the backward timed out.
void check_fwd_bwd_status(const Tensor& counts, const Tensor& status) {
    Tensor c = at::cat({counts.narrow(0, 0, 1), status}).to(at::kCPU);
    const int32_t* p = c.data_ptr<int32_t>();
    TORCH_CHECK(p[0] >= 0, "dot_sinkhorn_forward: a cross-workgroup exchange timed out (outputs are NaN)");
    TORCH_CHECK(p[1] == 0, "dot_sinkhorn_backward: a cross-workgroup exchange timed out (gradients are NaN)");
}

void check_grad_shape(const Tensor& log_alpha, const Tensor& grad_P) {
    check_hip_input(grad_P, "grad_P");
    TORCH_CHECK(grad_P.sizes() == log_alpha.sizes(), "grad_P must match log_alpha shape");
}

// sinkhorn_with_grads_unrolled (torch_cuda.cpp:717-801): forward with the u/v
// history, then the reverse pass -> [P, grad_log_alpha, grad_tau].
std::vector<Tensor> sinkhorn_with_grads_unrolled_op(Tensor log_alpha, Tensor grad_P, double tau,
                                                    int64_t n_iters, optional<Tensor> log_a,
                                                    optional<Tensor> log_b) {
    check_common(log_alpha, tau, n_iters);
    check_grad_shape(log_alpha, grad_P);
    check_marginals(log_a, log_b, log_alpha.size(0), log_alpha.size(1), log_alpha.size(2));
    c10::OptionalDeviceGuard guard(log_alpha.device());
    Tensor la = f32c(log_alpha);
    ForwardOut o = run_forward(la, DOT_SCORES_LOG_ALPHA, tau, n_iters, 0.0, f32c_opt(log_a),
                               f32c_opt(log_b), false, true, false, true);
    std::vector<Tensor> g = run_backward(false, la, DOT_SCORES_LOG_ALPHA, o.plan, f32c(grad_P),
                                         c10::nullopt, tau, n_iters, o.u_hist, o.v_hist);
    check_fwd_bwd_status(o.counts, g[2]);
    return {o.plan, g[0], g[1]};
}

// sinkhorn_with_grads_implicit (torch_cuda.cpp:803-871): forward with tol = 0,
// then at most backward_iters adjoint sweeps (exactly that many with
// DOT_AMD_EXACT_SWEEPS=1) -> [P, grad_log_alpha, grad_tau].
std::vector<Tensor> sinkhorn_with_grads_implicit_op(Tensor log_alpha, Tensor grad_P, double tau,
                                                    int64_t n_iters, int64_t backward_iters,
                                                    optional<Tensor> log_a, optional<Tensor> log_b) {
    check_common(log_alpha, tau, n_iters);
    check_grad_shape(log_alpha, grad_P);
    TORCH_CHECK(backward_iters >= 0, "backward_iters must be >= 0");
    check_marginals(log_a, log_b, log_alpha.size(0), log_alpha.size(1), log_alpha.size(2));
    c10::OptionalDeviceGuard guard(log_alpha.device());
    Tensor la = f32c(log_alpha);
    ForwardOut o = run_forward(la, DOT_SCORES_LOG_ALPHA, tau, n_iters, 0.0, f32c_opt(log_a),
                               f32c_opt(log_b), false, true, false, false);
    std::vector<Tensor> g = run_backward(true, la, DOT_SCORES_LOG_ALPHA, o.plan, f32c(grad_P),
                                         c10::nullopt, tau, backward_iters, Tensor(), Tensor());
    check_fwd_bwd_status(o.counts, g[2]);
    return {o.plan, g[0], g[1]};
}

void check_lengths(const Tensor& lengths, int64_t B) {
    check_hip_input(lengths, "lengths");
    TORCH_CHECK(lengths.dim() == 2 && lengths.size(1) == 2, "lengths must be [B, 2]");
    TORCH_CHECK(lengths.dtype() == at::kInt, "lengths must be int32");
    TORCH_CHECK(lengths.size(0) == B, "lengths must have one row per batch element");
}

// bidirectional_softmax (bidirectional_softmax/torch_cuda.cpp:42-76) -> [P, row_sm, col_sm].
std::vector<Tensor> bidirectional_softmax_op(Tensor sim, double tau, Tensor lengths) {
    check_hip_input(sim, "sim_matrix");
    TORCH_CHECK(sim.dim() == 3, "sim_matrix must be 3D [B, L1, L2]");
    check_lengths(lengths, sim.size(0));
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    c10::OptionalDeviceGuard guard(sim.device());
    Tensor s = f32c(sim);
    Tensor ln = lengths.contiguous();
    const int64_t B = s.size(0), L1 = s.size(1), L2 = s.size(2);
    auto opts = s.options();
    Tensor out = at::empty({B, L1, L2}, opts);
    Tensor r = at::empty({B, L1, L2}, opts);
    Tensor c = at::empty({B, L1, L2}, opts);
    const size_t ws_bytes = dot_bidisoftmax_forward_workspace_bytes(int(B), int(L1), int(L2));
    Tensor ws = workspace(ws_bytes, s);
    dot_bidisoftmax_fwd_args a{};
    a.sim = s.data_ptr<float>();
    a.lengths = ln.data_ptr<int32_t>();
    a.B = int(B);
    a.L1 = int(L1);
    a.L2 = int(L2);
    a.tau = static_cast<float>(tau);
    a.out = out.data_ptr<float>();
    a.row_sm = r.data_ptr<float>();
    a.col_sm = c.data_ptr<float>();
    a.workspace = ws.data_ptr();
    a.workspace_bytes = ws_bytes;
    check_rc(dot_bidisoftmax_forward(&a, current_stream(s)), "dot_bidisoftmax_forward");
    return {out, r, c};
}

std::vector<Tensor> bidi_backward_common(const Tensor& sim, const Tensor& grad_output, double tau,
                                         const Tensor& lengths, const Tensor& out, const Tensor& r,
                                         const Tensor& c, const Tensor& row_stats,
                                         const Tensor& col_stats, bool want_tau = true) {
    const int64_t B = sim.size(0), L1 = sim.size(1), L2 = sim.size(2);
    auto opts = sim.options();
    Tensor grad = at::empty({B, L1, L2}, opts);
    Tensor grad_tau = at::empty({want_tau ? B : 0}, opts);
    const size_t ws_bytes = dot_bidisoftmax_backward_workspace_bytes(int(B), int(L1), int(L2));
    Tensor ws = workspace(ws_bytes, sim);
    dot_bidisoftmax_bwd_args a{};
    a.sim = sim.data_ptr<float>();
    a.lengths = lengths.defined() ? lengths.data_ptr<int32_t>() : nullptr;
    a.B = int(B);
    a.L1 = int(L1);
    a.L2 = int(L2);
    a.tau = static_cast<float>(tau);
    a.grad_out = grad_output.data_ptr<float>();
    a.out = out.defined() ? out.data_ptr<float>() : nullptr;
    a.row_sm = r.defined() ? r.data_ptr<float>() : nullptr;
    a.col_sm = c.defined() ? c.data_ptr<float>() : nullptr;
    a.row_stats = row_stats.defined() ? row_stats.data_ptr<float>() : nullptr;
    a.col_stats = col_stats.defined() ? col_stats.data_ptr<float>() : nullptr;
    a.grad_sim = grad.data_ptr<float>();
    a.grad_tau = want_tau ? grad_tau.data_ptr<float>() : nullptr;
    a.workspace = ws.data_ptr();
    a.workspace_bytes = ws_bytes;
    std::tie(a.exchange, a.exchange_epoch) = bidi_exchange(sim);
    check_rc(dot_bidisoftmax_backward(&a, current_stream(sim)), "dot_bidisoftmax_backward");
    return {grad, grad_tau};
}

// bidirectional_softmax_backward (bidirectional_softmax/torch_cuda.cpp:78-139) -> [grad_sim, grad_tau].
std::vector<Tensor> bidirectional_softmax_backward_op(Tensor sim, Tensor output, Tensor grad_output,
                                                      Tensor row_softmax, Tensor col_softmax,
                                                      double tau, Tensor lengths) {
    for (auto* t : {&sim, &output, &grad_output, &row_softmax, &col_softmax})
        check_hip_input(*t, "bidirectional_softmax_backward inputs");
    TORCH_CHECK(sim.dim() == 3, "sim_matrix must be 3D [B, L1, L2]");
    TORCH_CHECK(output.sizes() == sim.sizes(), "output must match sim_matrix shape");
    TORCH_CHECK(grad_output.sizes() == sim.sizes(), "grad_output must match sim_matrix shape");
    TORCH_CHECK(row_softmax.sizes() == sim.sizes(), "row_softmax must match sim_matrix shape");
    TORCH_CHECK(col_softmax.sizes() == sim.sizes(), "col_softmax must match sim_matrix shape");
    check_lengths(lengths, sim.size(0));
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    c10::OptionalDeviceGuard guard(sim.device());
    return bidi_backward_common(f32c(sim), f32c(grad_output), tau, lengths.contiguous(), f32c(output),
                                f32c(row_softmax), f32c(col_softmax), Tensor(), Tensor());
}

// ---------------------------------------------------------------------------
// torch.ops.dot_amd.* fused operators (HIP only)
// ---------------------------------------------------------------------------

// -> [P, cost (B,) or undefined, counts int32[2] in pinned host memory (written by the
// forward's last kernel; read them once the stream has passed the call), u_hist, v_hist]
std::vector<Tensor> fused_forward_op(Tensor scores, int64_t scores_kind, double tau, int64_t n_iters,
                                     double tol, optional<Tensor> log_a, optional<Tensor> log_b,
                                     bool want_cost, bool keep_history) {
    check_common(scores, tau, n_iters);
    TORCH_CHECK(scores_kind == DOT_SCORES_LOG_ALPHA || scores_kind == DOT_SCORES_COST,
                "scores_kind must be 1 (log_alpha) or -1 (cost)");
    check_marginals(log_a, log_b, scores.size(0), scores.size(1), scores.size(2));
    c10::OptionalDeviceGuard guard(scores.device());
    ForwardOut o = run_forward(f32c(scores), int(scores_kind), tau, n_iters, tol, f32c_opt(log_a),
                               f32c_opt(log_b), false, true, want_cost, keep_history, /*counts_on_host=*/true);
    auto or_empty = [&](const Tensor& t) { return t.defined() ? t : at::empty({0}, scores.options().dtype(at::kFloat)); };
    return {o.plan, or_empty(o.cost), o.counts, or_empty(o.u_hist), or_empty(o.v_hist)};
}

// -> [plan, cost (B,) or empty, counts int32 [2]]
std::vector<Tensor> fused_forward_method_op(Tensor scores, int64_t scores_kind, double tau, int64_t n_iters,
                                            double tol, optional<Tensor> log_a, optional<Tensor> log_b,
                                            int64_t method, double omega, int64_t anderson_k,
                                            double mixing_beta, double lr, double beta1, double beta2,
                                            double eps_adam, bool bias_correction, double reg_start,
                                            int64_t schedule, bool want_cost) {
    check_common(scores, tau, n_iters);
    TORCH_CHECK(scores_kind == DOT_SCORES_LOG_ALPHA || scores_kind == DOT_SCORES_COST,
                "scores_kind must be 1 (log_alpha) or -1 (cost)");
    TORCH_CHECK(anderson_k >= 1, "anderson_k must be >= 1");
    check_marginals(log_a, log_b, scores.size(0), scores.size(1), scores.size(2));
    c10::OptionalDeviceGuard guard(scores.device());
    MethodParams mp{method, omega, anderson_k, mixing_beta, lr, beta1, beta2, eps_adam,
                    bias_correction, reg_start, schedule};
    ForwardOut o = run_forward_method(f32c(scores), int(scores_kind), tau, n_iters, tol, f32c_opt(log_a),
                                      f32c_opt(log_b), false, want_cost, mp);
    Tensor cost = o.cost.defined() ? o.cost : at::empty({0}, scores.options().dtype(at::kFloat));
    return {o.plan, cost, o.counts};
}

// -> [grad_scores, grad_tau (B,), status (int32 in pinned host memory, written
// by the backward's kernels: [0] is 1 when a cross-workgroup exchange timed
// out; implicit mode: [1 + b] the adjoint sweeps batch element b ran; read it
// after the stream has passed the call)]; mode 0 implicit (iters = adjoint
// sweeps at most), 1 unrolled (iters = T).
std::vector<Tensor> fused_backward_op(Tensor scores, int64_t scores_kind, Tensor plan,
                                      optional<Tensor> grad_plan, optional<Tensor> grad_cost,
                                      double tau, int64_t mode, int64_t iters,
                                      optional<Tensor> u_hist, optional<Tensor> v_hist, bool grad_cost_scalar) {
    check_hip_input(scores, "scores");
    check_hip_input(plan, "plan");
    TORCH_CHECK(scores.dim() == 3 && plan.sizes() == scores.sizes(), "plan must match scores");
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    TORCH_CHECK(iters >= 0, "iters must be >= 0");
    if (grad_plan.has_value()) TORCH_CHECK(grad_plan->sizes() == scores.sizes(), "grad_plan shape");
    if (grad_cost.has_value())
        TORCH_CHECK(grad_cost->dim() == 1 && grad_cost->size(0) == (grad_cost_scalar ? 1 : scores.size(0)),
                    "grad_cost shape");
    c10::OptionalDeviceGuard guard(scores.device());
    Tensor uh = u_hist.has_value() ? f32c(*u_hist) : Tensor();
    Tensor vh = v_hist.has_value() ? f32c(*v_hist) : Tensor();
    if (mode == 1 && iters > 0)
        TORCH_CHECK(uh.defined() && vh.defined() && uh.size(0) >= iters && vh.size(0) >= iters,
                    "unrolled backward needs the u/v history of every iteration");
    return run_backward(mode == 0, f32c(scores), int(scores_kind), f32c(plan), f32c_opt(grad_plan),
                        f32c_opt(grad_cost), tau, iters, uh, vh, /*status_on_host=*/true, grad_cost_scalar);
}

// -> [out, row_stats (B,2,L1), col_stats (B,2,L2)]; no lengths: every element full
std::vector<Tensor> bidi_forward_op(Tensor sim, double tau, optional<Tensor> lengths) {
    check_hip_input(sim, "sim_matrix");
    TORCH_CHECK(sim.dim() == 3, "sim_matrix must be 3D [B, L1, L2]");
    if (lengths.has_value()) check_lengths(*lengths, sim.size(0));
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    c10::OptionalDeviceGuard guard(sim.device());
    Tensor s = f32c(sim);
    Tensor ln = lengths.has_value() ? lengths->contiguous() : Tensor();
    const int64_t B = s.size(0), L1 = s.size(1), L2 = s.size(2);
    auto opts = s.options();
    Tensor out = at::empty({B, L1, L2}, opts);
    Tensor rs = at::empty({B, 2, L1}, opts);
    Tensor cs = at::empty({B, 2, L2}, opts);
    const size_t ws_bytes = dot_bidisoftmax_forward_workspace_bytes(int(B), int(L1), int(L2));
    Tensor ws = workspace(ws_bytes, s);
    dot_bidisoftmax_fwd_args a{};
    a.sim = s.data_ptr<float>();
    a.lengths = ln.defined() ? ln.data_ptr<int32_t>() : nullptr;
    a.B = int(B);
    a.L1 = int(L1);
    a.L2 = int(L2);
    a.tau = static_cast<float>(tau);
    a.out = out.data_ptr<float>();
    a.row_stats = rs.data_ptr<float>();
    a.col_stats = cs.data_ptr<float>();
    a.workspace = ws.data_ptr();
    a.workspace_bytes = ws_bytes;
    std::tie(a.exchange, a.exchange_epoch) = bidi_exchange(s);
    check_rc(dot_bidisoftmax_forward(&a, current_stream(s)), "dot_bidisoftmax_forward");
    return {out, rs, cs};
}

std::vector<Tensor> bidi_backward_op(Tensor sim, Tensor grad_output, Tensor row_stats,
                                     Tensor col_stats, double tau, optional<Tensor> lengths) {
    for (auto* t : {&sim, &grad_output, &row_stats, &col_stats}) check_hip_input(*t, "inputs");
    TORCH_CHECK(sim.dim() == 3 && grad_output.sizes() == sim.sizes(), "grad_output must match sim");
    if (lengths.has_value()) check_lengths(*lengths, sim.size(0));
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    c10::OptionalDeviceGuard guard(sim.device());
    // the autograd path has no tau gradient (the reference drops it): grad_tau is skipped
    return bidi_backward_common(f32c(sim), f32c(grad_output), tau,
                                lengths.has_value() ? lengths->contiguous() : Tensor(), Tensor(), Tensor(), Tensor(),
                                f32c(row_stats), f32c(col_stats), false);
}

}  // namespace

TORCH_LIBRARY(dot, m) {
    m.def("sinkhorn(Tensor log_alpha, float tau, int n_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor");
    m.def("sinkhorn_log(Tensor log_alpha, float tau, int n_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor");
    m.def(
        "sinkhorn_dual_forward("
        "Tensor log_alpha, float tau, int n_iters, float tol=0.0, Tensor? log_a=None, Tensor? log_b=None, "
        "bool return_log=False, int method=0, float omega=1.5, int anderson_k=5, float mixing_beta=1.0, "
        "float lr=1.0, float beta1=0.9, float beta2=0.999, float eps_adam=1e-8, bool bias_correction=True, "
        "float reg_start=-1.0, int schedule=0"
        ") -> Tensor[]");
    m.def("sinkhorn_spectral_preflight(Tensor log_alpha, float tau, int n_power=8) -> Tensor");
    m.def("sinkhorn_with_grads_unrolled(Tensor log_alpha, Tensor grad_P, float tau, int n_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor[]");
    m.def("sinkhorn_with_grads_implicit(Tensor log_alpha, Tensor grad_P, float tau, int n_iters, int backward_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor[]");
    m.def("bidirectional_softmax(Tensor sim, float tau, Tensor lengths) -> Tensor[]");
    m.def("bidirectional_softmax_backward(Tensor sim, Tensor output, Tensor grad_output, Tensor row_softmax, Tensor col_softmax, float tau, Tensor lengths) -> Tensor[]");
}

TORCH_LIBRARY_IMPL(dot, CUDA, m) {
    m.impl("sinkhorn", sinkhorn_op);
    m.impl("sinkhorn_log", sinkhorn_log_op);
    m.impl("sinkhorn_dual_forward", sinkhorn_dual_forward_op);
    m.impl("sinkhorn_spectral_preflight", sinkhorn_spectral_preflight_op);
    m.impl("sinkhorn_with_grads_unrolled", sinkhorn_with_grads_unrolled_op);
    m.impl("sinkhorn_with_grads_implicit", sinkhorn_with_grads_implicit_op);
    m.impl("bidirectional_softmax", bidirectional_softmax_op);
    m.impl("bidirectional_softmax_backward", bidirectional_softmax_backward_op);
}

TORCH_LIBRARY(dot_amd, m) {
    m.def("sinkhorn_forward(Tensor scores, int scores_kind, float tau, int n_iters, float tol, Tensor? log_a, Tensor? log_b, bool want_cost, bool keep_history) -> Tensor[]");
    m.def("sinkhorn_forward_method(Tensor scores, int scores_kind, float tau, int n_iters, float tol, Tensor? log_a, Tensor? log_b, int method, float omega, int anderson_k, float mixing_beta, float lr, float beta1, float beta2, float eps_adam, bool bias_correction, float reg_start, int schedule, bool want_cost) -> Tensor[]");
    m.def("sinkhorn_backward(Tensor scores, int scores_kind, Tensor plan, Tensor? grad_plan, Tensor? grad_cost, float tau, int mode, int iters, Tensor? u_hist, Tensor? v_hist, bool grad_cost_scalar=False) -> Tensor[]");
    m.def("bidirectional_softmax_forward(Tensor sim, float tau, Tensor? lengths) -> Tensor[]");
    m.def("bidirectional_softmax_backward(Tensor sim, Tensor grad_output, Tensor row_stats, Tensor col_stats, float tau, Tensor? lengths) -> Tensor[]");
}

TORCH_LIBRARY_IMPL(dot_amd, CUDA, m) {
    m.impl("sinkhorn_forward", fused_forward_op);
    m.impl("sinkhorn_forward_method", fused_forward_method_op);
    m.impl("sinkhorn_backward", fused_backward_op);
    m.impl("bidirectional_softmax_forward", bidi_forward_op);
    m.impl("bidirectional_softmax_backward", bidi_backward_op);
}
