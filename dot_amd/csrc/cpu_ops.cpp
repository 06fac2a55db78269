// CPU implementations of the eight torch.ops.dot operators, registered under
// the CPU dispatch key: the reference's src/sinkhorn/torch_cpu.cpp:23-328 and
// src/bidirectional_softmax/torch_cpu.cpp:22-111 with their semantics
// (sinkhorn_dual_forward ignores tol and method, reports n_iters and
// converged = tol <= 0; the implicit adjoint stops at max change < 1e-6;
// K = log_alpha / tau; safe_exp throughout).
//
// Design: the Sinkhorn iteration runs in dual form — the scaled scores K of a
// batch element are computed once and two potentials u, v carry the
// iteration — instead of rewriting log P in place twice per iteration as the
// reference does.  It is the same iteration (log P = K + u + v after every
// half-step); the potentials round once per step instead of every entry of
// log P, sums accumulate in double, and the column log-sum-exp is a row-major
// online (max, sum) pass over fixed chunks of rows merged in chunk order, so
// the matrix is never walked down a column and results do not depend on the
// thread count.  The unrolled backward keeps the potentials of every
// iteration (T (n + m) floats) and recomputes the reference's exp(X_t),
// exp(Y_t) from them, where the reference stores T + 1 full matrices.  Batch
// elements, rows and row chunks run in parallel (at::parallel_for).
#include <ATen/ATen.h>
#include <ATen/Parallel.h>
#include <torch/library.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <vector>

namespace {

using at::Tensor;
using c10::optional;

constexpr int64_t kChunkRows = 32;  // rows per column-partial chunk (fixed: results independent of threads)
constexpr float kDenFloor = 1.0e-12f;

inline float safe_exp(float x) {  // kernels_cpu.cpp:18-22
    if (x < -88.0f) return 0.0f;
    return std::exp(std::min(x, 88.0f));
}

void check_cpu(const Tensor& t, const char* name) {
    TORCH_CHECK(t.device().is_cpu(), name, " must be a CPU tensor");
}

void check_marginals(const optional<Tensor>& log_a, const optional<Tensor>& log_b, int64_t B, int64_t n,
                     int64_t m) {
    if (log_a.has_value()) {
        check_cpu(*log_a, "log_a");
        TORCH_CHECK(log_a->dim() == 2 && log_a->size(0) == B && log_a->size(1) == n, "log_a must have shape [B, n]");
    }
    if (log_b.has_value()) {
        check_cpu(*log_b, "log_b");
        TORCH_CHECK(log_b->dim() == 2 && log_b->size(0) == B && log_b->size(1) == m, "log_b must have shape [B, m]");
    }
}

void check_common(const Tensor& log_alpha, double tau, int64_t n_iters) {
    check_cpu(log_alpha, "log_alpha");
    TORCH_CHECK(log_alpha.dim() == 3, "log_alpha must be 3D [B, n, m]");
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    TORCH_CHECK(n_iters >= 0, "n_iters must be >= 0");
}

Tensor f32c(const Tensor& t) { return t.to(at::kFloat).contiguous(); }
optional<Tensor> f32c_opt(const optional<Tensor>& t) {
    if (!t.has_value()) return c10::nullopt;
    return f32c(*t);
}

// log-sum-exp of a row of `len` values y_j = a_j + b_j (kernels_cpu.cpp:28-52:
// max from -FLT_MAX; -FLT_MAX for an empty or all -inf row).
inline float row_lse(const float* a, const float* b, int64_t len) {
    float mx = -FLT_MAX;
    for (int64_t j = 0; j < len; ++j) mx = std::max(mx, a[j] + (b ? b[j] : 0.0f));
    if (mx == -FLT_MAX) return -FLT_MAX;
    double s = 0.0;
    for (int64_t j = 0; j < len; ++j) s += safe_exp(a[j] + (b ? b[j] : 0.0f) - mx);
    if (s == 0.0) return -FLT_MAX;
    return mx + static_cast<float>(std::log(s));
}

// One batch element of the dual iteration.
struct Element {
    int64_t n, m;
    std::vector<float> K;  // [n, m] = log_alpha / tau
    std::vector<float> u, v;
    const float* log_a;    // [n] or null (-log n)
    const float* log_b;    // [m] or null (-log m)

    Element(const float* la, float tau, int64_t n_, int64_t m_, const float* lga, const float* lgb)
        : n(n_), m(m_), K(static_cast<size_t>(n_ * m_)), u(size_t(n_), 0.0f), v(size_t(m_), 0.0f), log_a(lga), log_b(lgb) {
        for (int64_t k = 0; k < n * m; ++k) K[size_t(k)] = la[k] / tau;  // kernels_cpu.cpp:78-80
    }

    float target_a(int64_t i) const { return log_a ? log_a[i] : -std::log(static_cast<float>(n)); }
    float target_b(int64_t j) const { return log_b ? log_b[j] : -std::log(static_cast<float>(m)); }

    // u_i = log a_i - LSE_j(K_ij + v_j)
    void row_update() {
        at::parallel_for(0, n, 16, [&](int64_t i0, int64_t i1) {
            for (int64_t i = i0; i < i1; ++i)
                u[size_t(i)] = target_a(i) - row_lse(K.data() + i * m, v.data(), m);
        });
    }

    // v_j = log b_j - LSE_i(K_ij + u_i): per chunk of rows an online (max, sum)
    // per column, merged in chunk order.
    void col_update() {
        const int64_t nchunk = (n + kChunkRows - 1) / kChunkRows;
        std::vector<float> cmax(static_cast<size_t>(nchunk * m));
        std::vector<double> csum(static_cast<size_t>(nchunk * m));
        at::parallel_for(0, nchunk, 1, [&](int64_t c0, int64_t c1) {
            for (int64_t c = c0; c < c1; ++c) {
                float* mx = cmax.data() + c * m;
                double* s = csum.data() + c * m;
                std::fill(mx, mx + m, -FLT_MAX);
                std::fill(s, s + m, 0.0);
                const int64_t r1 = std::min(n, (c + 1) * kChunkRows);
                for (int64_t i = c * kChunkRows; i < r1; ++i) {
                    const float* k = K.data() + i * m;
                    const float ui = u[size_t(i)];
                    for (int64_t j = 0; j < m; ++j) {
                        const float y = k[j] + ui;
                        if (y > mx[j]) {
                            s[j] = s[j] * safe_exp(mx[j] - y) + 1.0;
                            mx[j] = y;
                        } else {
                            s[j] += safe_exp(y - mx[j]);
                        }
                    }
                }
            }
        });
        at::parallel_for(0, m, 256, [&](int64_t j0, int64_t j1) {
            for (int64_t j = j0; j < j1; ++j) {
                float M = -FLT_MAX;
                for (int64_t c = 0; c < nchunk; ++c) M = std::max(M, cmax[size_t(c * m + j)]);
                double S = 0.0;
                if (M != -FLT_MAX)
                    for (int64_t c = 0; c < nchunk; ++c)
                        S += csum[size_t(c * m + j)] * safe_exp(cmax[size_t(c * m + j)] - M);
                const float lse = (M == -FLT_MAX || S == 0.0) ? -FLT_MAX : M + static_cast<float>(std::log(S));
                v[size_t(j)] = target_b(j) - lse;
            }
        });
    }

    float logp(int64_t i, int64_t j) const { return K[size_t(i * m + j)] + u[size_t(i)] + v[size_t(j)]; }
};

// Runs f(b) for every batch element: elements in parallel when there are
// several, each element's own loops in parallel otherwise.
template <class F>
void for_each_element(int64_t B, F&& f) {
    if (B <= 1) {
        for (int64_t b = 0; b < B; ++b) f(b);
    } else {
        at::parallel_for(0, B, 1, [&](int64_t b0, int64_t b1) {
            for (int64_t b = b0; b < b1; ++b) f(b);
        });
    }
}

const float* row_of(const optional<Tensor>& t, int64_t b, int64_t len) {
    return t.has_value() ? t->data_ptr<float>() + b * len : nullptr;
}

// Forward of sinkhorn / sinkhorn_log (sinkhorn_forward_cpu, kernels_cpu.cpp:60-107).
Tensor forward_cpu(const Tensor& la_f, double tau, int64_t n_iters, const optional<Tensor>& lga,
                   const optional<Tensor>& lgb, bool return_log, std::vector<float>* u_hist = nullptr,
                   std::vector<float>* v_hist = nullptr) {
    const int64_t B = la_f.size(0), n = la_f.size(1), m = la_f.size(2);
    Tensor out = at::empty({B, n, m}, la_f.options());
    const float* la = la_f.data_ptr<float>();
    float* o = out.data_ptr<float>();
    for_each_element(B, [&](int64_t b) {
        Element e(la + b * n * m, static_cast<float>(tau), n, m, row_of(lga, b, n), row_of(lgb, b, m));
        for (int64_t t = 0; t < n_iters; ++t) {
            e.row_update();
            e.col_update();
            if (u_hist) {
                std::copy(e.u.begin(), e.u.end(), u_hist->begin() + (t * B + b) * n);
                std::copy(e.v.begin(), e.v.end(), v_hist->begin() + (t * B + b) * m);
            }
        }
        float* ob = o + b * n * m;
        at::parallel_for(0, n, 16, [&](int64_t i0, int64_t i1) {
            for (int64_t i = i0; i < i1; ++i)
                for (int64_t j = 0; j < m; ++j) {
                    const float lp = e.logp(i, j);
                    ob[i * m + j] = return_log ? lp : safe_exp(lp);
                }
        });
    });
    return out;
}

Tensor sinkhorn_cpu(Tensor log_alpha, double tau, int64_t n_iters, optional<Tensor> log_a, optional<Tensor> log_b) {
    check_common(log_alpha, tau, n_iters);
    check_marginals(log_a, log_b, log_alpha.size(0), log_alpha.size(1), log_alpha.size(2));
    return forward_cpu(f32c(log_alpha), tau, n_iters, f32c_opt(log_a), f32c_opt(log_b), false);
}

Tensor sinkhorn_log_cpu(Tensor log_alpha, double tau, int64_t n_iters, optional<Tensor> log_a,
                        optional<Tensor> log_b) {
    check_common(log_alpha, tau, n_iters);
    check_marginals(log_a, log_b, log_alpha.size(0), log_alpha.size(1), log_alpha.size(2));
    return forward_cpu(f32c(log_alpha), tau, n_iters, f32c_opt(log_a), f32c_opt(log_b), true);
}

// torch_cpu.cpp:115-151: the CPU op runs the plain forward for n_iters
// iterations whatever tol and method say.
std::vector<Tensor> sinkhorn_dual_forward_cpu(Tensor log_alpha, double tau, int64_t n_iters, double tol,
                                              optional<Tensor> log_a, optional<Tensor> log_b, bool return_log,
                                              int64_t, double, int64_t, double, double, double, double, double,
                                              bool, double, int64_t) {
    check_common(log_alpha, tau, n_iters);
    check_marginals(log_a, log_b, log_alpha.size(0), log_alpha.size(1), log_alpha.size(2));
    Tensor P = forward_cpu(f32c(log_alpha), tau, n_iters, f32c_opt(log_a), f32c_opt(log_b), return_log);
    auto opt = at::TensorOptions().dtype(at::kLong).device(at::kCPU);
    return {P, at::scalar_tensor(n_iters, opt), at::scalar_tensor(int64_t(tol <= 0.0 ? 1 : 0), opt)};
}

// Implicit backward (sinkhorn_backward_implicit_cpu, kernels_cpu.cpp:247-327):
// Gauss-Seidel sweeps lambda then mu, stopping once the largest change is
// below 1e-6 (torch_cpu.cpp:318), then grad = P (G - lambda - mu) / tau and
// grad_tau = -sum(grad * log_alpha) / tau.
std::vector<Tensor> with_grads_implicit_cpu(Tensor log_alpha, Tensor grad_P, double tau, int64_t n_iters,
                                            int64_t backward_iters, optional<Tensor> log_a, optional<Tensor> log_b) {
    check_common(log_alpha, tau, n_iters);
    check_cpu(grad_P, "grad_P");
    TORCH_CHECK(grad_P.sizes() == log_alpha.sizes(), "grad_P must match log_alpha shape");
    TORCH_CHECK(backward_iters >= 0, "backward_iters must be >= 0");
    const int64_t B = log_alpha.size(0), n = log_alpha.size(1), m = log_alpha.size(2);
    check_marginals(log_a, log_b, B, n, m);
    Tensor la_f = f32c(log_alpha), G_f = f32c(grad_P);
    Tensor P = forward_cpu(la_f, tau, n_iters, f32c_opt(log_a), f32c_opt(log_b), false);
    Tensor grad = at::empty({B, n, m}, la_f.options());
    Tensor grad_tau = at::empty({B}, la_f.options());
    const float* la = la_f.data_ptr<float>();
    const float* Gp = G_f.data_ptr<float>();
    const float* Pp = P.data_ptr<float>();
    float* gp = grad.data_ptr<float>();
    float* gt = grad_tau.data_ptr<float>();
    const float ftau = static_cast<float>(tau);
    for_each_element(B, [&](int64_t b) {
        const float* Pb = Pp + b * n * m;
        const float* Gb = Gp + b * n * m;
        // the constant sums of every sweep: sum P G and sum P per row and per column
        std::vector<double> rPG(static_cast<size_t>(n)), rP(static_cast<size_t>(n)), cPG(static_cast<size_t>(m), 0.0), cP(static_cast<size_t>(m), 0.0);
        for (int64_t i = 0; i < n; ++i) {
            double a = 0.0, c = 0.0;
            for (int64_t k = 0; k < m; ++k) {
                const double p = Pb[i * m + k];
                a += p * Gb[i * m + k];
                c += p;
                cPG[size_t(k)] += p * Gb[i * m + k];
                cP[size_t(k)] += p;
            }
            rPG[size_t(i)] = a;
            rP[size_t(i)] = c;
        }
        std::vector<float> lam(static_cast<size_t>(n), 0.0f), mu(size_t(m), 0.0f);
        std::vector<double> pl(static_cast<size_t>(m));
        for (int64_t it = 0; it < backward_iters; ++it) {
            float change = 0.0f;
            for (int64_t i = 0; i < n; ++i) {
                double pm = 0.0;
                for (int64_t k = 0; k < m; ++k) pm += double(Pb[i * m + k]) * mu[size_t(k)];
                const float nl = float((rPG[size_t(i)] - pm) / std::max(rP[size_t(i)], double(kDenFloor)));
                change = std::max(change, std::abs(nl - lam[size_t(i)]));
                lam[size_t(i)] = nl;
            }
            std::fill(pl.begin(), pl.end(), 0.0);
            for (int64_t i = 0; i < n; ++i)
                for (int64_t k = 0; k < m; ++k) pl[size_t(k)] += double(Pb[i * m + k]) * lam[size_t(i)];
            for (int64_t k = 0; k < m; ++k) {
                const float nm = float((cPG[size_t(k)] - pl[size_t(k)]) / std::max(cP[size_t(k)], double(kDenFloor)));
                change = std::max(change, std::abs(nm - mu[size_t(k)]));
                mu[size_t(k)] = nm;
            }
            if (change < 1.0e-6f) break;
        }
        double gsum = 0.0;
        float* gb = gp + b * n * m;
        const float* lab = la + b * n * m;
        for (int64_t i = 0; i < n; ++i)
            for (int64_t k = 0; k < m; ++k) {
                const float g = Pb[i * m + k] * (Gb[i * m + k] - lam[size_t(i)] - mu[size_t(k)]) / ftau;
                gb[i * m + k] = g;
                gsum += double(g) * lab[i * m + k];
            }
        gt[b] = float(-gsum / tau);
    });
    return {P, grad, grad_tau};
}

// Unrolled backward (sinkhorn_backward_unrolled_cpu, kernels_cpu.cpp:169-245)
// from the potentials: X_t = K + u_t + v_t after t iterations, Y_t = K +
// u_{t+1} + v_t after the row half-step of iteration t+1; Gamma = grad_P * P,
// then for t = T-1..0: Gamma_Y = Gamma - exp(X_{t+1}) colsum(Gamma),
// Gamma = Gamma_Y - exp(Y_t) rowsum(Gamma_Y); grad = Gamma / tau,
// grad_tau = -sum(Gamma * log_alpha) / tau^2.
std::vector<Tensor> with_grads_unrolled_cpu(Tensor log_alpha, Tensor grad_P, double tau, int64_t n_iters,
                                            optional<Tensor> log_a, optional<Tensor> log_b) {
    check_common(log_alpha, tau, n_iters);
    check_cpu(grad_P, "grad_P");
    TORCH_CHECK(grad_P.sizes() == log_alpha.sizes(), "grad_P must match log_alpha shape");
    const int64_t B = log_alpha.size(0), n = log_alpha.size(1), m = log_alpha.size(2);
    check_marginals(log_a, log_b, B, n, m);
    Tensor la_f = f32c(log_alpha), G_f = f32c(grad_P);
    std::vector<float> uh(static_cast<size_t>(n_iters * B * n)), vh(static_cast<size_t>(n_iters * B * m));
    Tensor P = forward_cpu(la_f, tau, n_iters, f32c_opt(log_a), f32c_opt(log_b), false, &uh, &vh);
    Tensor grad = at::empty({B, n, m}, la_f.options());
    Tensor grad_tau = at::empty({B}, la_f.options());
    const float* la = la_f.data_ptr<float>();
    const float* Gp = G_f.data_ptr<float>();
    const float* Pp = P.data_ptr<float>();
    float* gp = grad.data_ptr<float>();
    float* gt = grad_tau.data_ptr<float>();
    const float ftau = static_cast<float>(tau);
    for_each_element(B, [&](int64_t b) {
        const float* lab = la + b * n * m;
        std::vector<float> K(static_cast<size_t>(n * m));
        for (int64_t k = 0; k < n * m; ++k) K[size_t(k)] = lab[k] / ftau;
        std::vector<float> Gam(static_cast<size_t>(n * m));
        for (int64_t k = 0; k < n * m; ++k) Gam[size_t(k)] = Gp[b * n * m + k] * Pp[b * n * m + k];
        std::vector<double> cs(static_cast<size_t>(m));
        std::vector<float> zero_v(static_cast<size_t>(m), 0.0f);
        for (int64_t t = n_iters - 1; t >= 0; --t) {
            const float* u1 = uh.data() + (t * B + b) * n;                           // u_{t+1}
            const float* v1 = vh.data() + (t * B + b) * m;                           // v_{t+1}
            const float* v0 = t > 0 ? vh.data() + ((t - 1) * B + b) * m : zero_v.data();  // v_t
            std::fill(cs.begin(), cs.end(), 0.0);
            for (int64_t i = 0; i < n; ++i)
                for (int64_t k = 0; k < m; ++k) cs[size_t(k)] += Gam[size_t(i * m + k)];
            at::parallel_for(0, n, 16, [&](int64_t i0, int64_t i1) {
                for (int64_t i = i0; i < i1; ++i) {
                    float* g = Gam.data() + i * m;
                    const float* kr = K.data() + i * m;
                    double rs = 0.0;
                    for (int64_t k = 0; k < m; ++k) {
                        g[k] = g[k] - safe_exp(kr[k] + u1[i] + v1[k]) * float(cs[size_t(k)]);
                        rs += g[k];
                    }
                    const float r = float(rs);
                    for (int64_t k = 0; k < m; ++k) g[k] = g[k] - safe_exp(kr[k] + u1[i] + v0[k]) * r;
                }
            });
        }
        double gsum = 0.0;
        float* gb = gp + b * n * m;
        for (int64_t k = 0; k < n * m; ++k) {
            gb[k] = Gam[size_t(k)] / ftau;
            gsum += double(Gam[size_t(k)]) * lab[k];
        }
        gt[b] = float(-gsum / (tau * tau));
    });
    return {P, grad, grad_tau};
}

// Spectral preflight.  The reference's CPU op starts from an unseeded randn
// vector (torch_cpu.cpp:171); this one runs the GPU kernel's algorithm
// (kernels.cu:141-241) with its deterministic start vector, so CPU and HIP
// tensors give the same estimate: P = softmax_row(log_alpha / tau), v0_j =
// sin((j+1) 12.9898 + (b+1) 78.233) centred and normalised, n_power rounds of
// u = centre(P v), v = centre_normalise(P^T u), then ||centre(P v)|| clamped
// to [0, 0.999999].
Tensor spectral_preflight_cpu(Tensor log_alpha, double tau, int64_t n_power) {
    check_cpu(log_alpha, "log_alpha");
    TORCH_CHECK(log_alpha.dim() == 3, "log_alpha must be 3D [B, n, m]");
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    TORCH_CHECK(n_power >= 1, "n_power must be >= 1");
    Tensor la_f = f32c(log_alpha);
    const int64_t B = la_f.size(0), n = la_f.size(1), m = la_f.size(2);
    Tensor est = at::empty({B}, la_f.options());
    const float* la = la_f.data_ptr<float>();
    float* ep = est.data_ptr<float>();
    const float inv_tau = 1.0f / static_cast<float>(tau);
    auto centre_normalise = [](std::vector<double>& x) {
        double s = 0.0;
        for (double q : x) s += q;
        const double mean = x.empty() ? 0.0 : s / double(x.size());
        double ss = 0.0;
        for (double& q : x) {
            q -= mean;
            ss += q * q;
        }
        const double norm = std::sqrt(std::max(ss, 1.0e-12));
        for (double& q : x) q /= norm;
    };
    for_each_element(B, [&](int64_t b) {
        const float* lab = la + b * n * m;
        std::vector<float> P(static_cast<size_t>(n * m));
        for (int64_t i = 0; i < n; ++i) {
            const float* r = lab + i * m;
            float mx = -FLT_MAX;
            for (int64_t j = 0; j < m; ++j) mx = std::max(mx, r[j] * inv_tau);
            double s = 0.0;
            for (int64_t j = 0; j < m; ++j) s += safe_exp(r[j] * inv_tau - mx);
            const float lse = mx + float(std::log(std::max(s, double(kDenFloor))));
            for (int64_t j = 0; j < m; ++j) P[size_t(i * m + j)] = safe_exp(r[j] * inv_tau - lse);
        }
        std::vector<double> v(static_cast<size_t>(m)), u(static_cast<size_t>(n));
        for (int64_t j = 0; j < m; ++j) {
            const float t1 = static_cast<float>(j + 1) * 12.9898f;
            const float t2 = static_cast<float>(b + 1) * 78.233f;
            const float arg = t1 + t2;
            v[size_t(j)] = std::sin(arg);
        }
        centre_normalise(v);
        auto Pv = [&]() {
            double s = 0.0;
            for (int64_t i = 0; i < n; ++i) {
                double d = 0.0;
                for (int64_t j = 0; j < m; ++j) d += double(P[size_t(i * m + j)]) * v[size_t(j)];
                u[size_t(i)] = d;
                s += d;
            }
            const double mean = n ? s / double(n) : 0.0;
            for (double& q : u) q -= mean;
        };
        for (int64_t it = 0; it < n_power; ++it) {
            Pv();
            std::fill(v.begin(), v.end(), 0.0);
            for (int64_t i = 0; i < n; ++i)
                for (int64_t j = 0; j < m; ++j) v[size_t(j)] += double(P[size_t(i * m + j)]) * u[size_t(i)];
            centre_normalise(v);
        }
        Pv();
        double ss = 0.0;
        for (double q : u) ss += q * q;
        ep[b] = float(std::min(std::max(std::sqrt(std::max(ss, 1.0e-12)), 0.0), 0.999999));
    });
    return est;
}

// ---------------------------------------------------------------------------
// Bidirectional softmax (bidirectional_softmax/kernels_cpu.cpp:41-232)
// ---------------------------------------------------------------------------
constexpr float kBidiEps = 1.0e-9f;

void check_lengths(const Tensor& lengths, int64_t B) {
    check_cpu(lengths, "lengths");
    TORCH_CHECK(lengths.dim() == 2 && lengths.size(1) == 2, "lengths must be [B, 2]");
    TORCH_CHECK(lengths.dtype() == at::kInt, "lengths must be int32");
    TORCH_CHECK(lengths.size(0) == B, "lengths must have one row per batch element");
}

// valid extent of element b, clamped to the tensor (the reference reads past it)
inline void extent(const int32_t* ln, int64_t b, int64_t L1, int64_t L2, int64_t& l1, int64_t& l2) {
    l1 = std::min<int64_t>(std::max<int32_t>(ln[2 * b], 0), L1);
    l2 = std::min<int64_t>(std::max<int32_t>(ln[2 * b + 1], 0), L2);
}

// -> [out, row_softmax, col_softmax]; r and c are 0 outside the valid region.
std::vector<Tensor> bidirectional_softmax_cpu(Tensor sim, double tau, Tensor lengths) {
    check_cpu(sim, "sim_matrix");
    TORCH_CHECK(sim.dim() == 3, "sim_matrix must be 3D [B, L1, L2]");
    check_lengths(lengths, sim.size(0));
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    Tensor s = f32c(sim);
    Tensor ln = lengths.contiguous();
    const int64_t B = s.size(0), L1 = s.size(1), L2 = s.size(2);
    Tensor out = at::zeros({B, L1, L2}, s.options());
    Tensor rsm = at::zeros({B, L1, L2}, s.options());
    Tensor csm = at::zeros({B, L1, L2}, s.options());
    const float* sp = s.data_ptr<float>();
    const int32_t* lp = ln.data_ptr<int32_t>();
    float *op = out.data_ptr<float>(), *rp = rsm.data_ptr<float>(), *cp = csm.data_ptr<float>();
    const float inv_t = 1.0f / static_cast<float>(tau);
    for_each_element(B, [&](int64_t b) {
        int64_t l1, l2;
        extent(lp, b, L1, L2, l1, l2);
        const size_t base = size_t(b) * L1 * L2;
        const float* S = sp + base;
        float *R = rp + base, *Cm = cp + base, *O = op + base;
        at::parallel_for(0, l1, 16, [&](int64_t i0, int64_t i1) {
            for (int64_t i = i0; i < i1; ++i) {
                float mx = -1.0e30f;
                for (int64_t j = 0; j < l2; ++j) mx = std::max(mx, S[i * L2 + j] * inv_t);
                double sum = 0.0;
                for (int64_t j = 0; j < l2; ++j) {
                    const float e = safe_exp(S[i * L2 + j] * inv_t - mx);
                    R[i * L2 + j] = e;
                    sum += e;
                }
                if (sum > 0.0) {
                    const float inv = 1.0f / float(sum);
                    for (int64_t j = 0; j < l2; ++j) R[i * L2 + j] *= inv;
                }
            }
        });
        // columns: max and sum per column in a row-major pass
        std::vector<float> cmx(static_cast<size_t>(l2), -1.0e30f);
        std::vector<double> csum(static_cast<size_t>(l2), 0.0);
        for (int64_t i = 0; i < l1; ++i)
            for (int64_t j = 0; j < l2; ++j) cmx[size_t(j)] = std::max(cmx[size_t(j)], S[i * L2 + j] * inv_t);
        for (int64_t i = 0; i < l1; ++i)
            for (int64_t j = 0; j < l2; ++j) {
                const float e = safe_exp(S[i * L2 + j] * inv_t - cmx[size_t(j)]);
                Cm[i * L2 + j] = e;
                csum[size_t(j)] += e;
            }
        std::vector<float> cinv(static_cast<size_t>(l2), 1.0f);
        for (int64_t j = 0; j < l2; ++j) cinv[size_t(j)] = csum[size_t(j)] > 0.0 ? 1.0f / float(csum[size_t(j)]) : 1.0f;
        at::parallel_for(0, l1, 16, [&](int64_t i0, int64_t i1) {
            for (int64_t i = i0; i < i1; ++i)
                for (int64_t j = 0; j < l2; ++j) {
                    Cm[i * L2 + j] *= cinv[size_t(j)];
                    O[i * L2 + j] = std::sqrt(kBidiEps + R[i * L2 + j] * Cm[i * L2 + j]);
                }
        });
    });
    return {out, rsm, csm};
}

// -> [grad_sim, grad_tau]; d = g / (2 out) where out > 1e-9, then the row and
// column softmax backward; grad_tau = -sum(grad_sim * sim) / tau.
std::vector<Tensor> bidirectional_softmax_backward_cpu(Tensor sim, Tensor output, Tensor grad_output,
                                                       Tensor row_softmax, Tensor col_softmax, double tau,
                                                       Tensor lengths) {
    for (const Tensor* t : {&sim, &output, &grad_output, &row_softmax, &col_softmax}) check_cpu(*t, "inputs");
    TORCH_CHECK(sim.dim() == 3, "sim_matrix must be 3D [B, L1, L2]");
    TORCH_CHECK(output.sizes() == sim.sizes(), "output must match sim_matrix shape");
    TORCH_CHECK(grad_output.sizes() == sim.sizes(), "grad_output must match sim_matrix shape");
    TORCH_CHECK(row_softmax.sizes() == sim.sizes(), "row_softmax must match sim_matrix shape");
    TORCH_CHECK(col_softmax.sizes() == sim.sizes(), "col_softmax must match sim_matrix shape");
    check_lengths(lengths, sim.size(0));
    TORCH_CHECK(tau > 0.0, "tau must be > 0");
    Tensor s = f32c(sim), o = f32c(output), g = f32c(grad_output), r = f32c(row_softmax), c = f32c(col_softmax);
    Tensor ln = lengths.contiguous();
    const int64_t B = s.size(0), L1 = s.size(1), L2 = s.size(2);
    Tensor grad = at::zeros({B, L1, L2}, s.options());
    Tensor grad_tau = at::zeros({B}, s.options());
    const int32_t* lp = ln.data_ptr<int32_t>();
    const float inv_t = 1.0f / static_cast<float>(tau);
    for_each_element(B, [&](int64_t b) {
        int64_t l1, l2;
        extent(lp, b, L1, L2, l1, l2);
        const size_t base = size_t(b) * L1 * L2;
        const float *S = s.data_ptr<float>() + base, *O = o.data_ptr<float>() + base;
        const float *Gd = g.data_ptr<float>() + base, *R = r.data_ptr<float>() + base;
        const float* Cm = c.data_ptr<float>() + base;
        float* GS = grad.data_ptr<float>() + base;
        auto dprod = [&](int64_t idx) { return O[idx] > kBidiEps ? Gd[idx] * 0.5f / O[idx] : 0.0f; };
        // row part: (d c - sum_j d c r) r / tau
        at::parallel_for(0, l1, 16, [&](int64_t i0, int64_t i1) {
            for (int64_t i = i0; i < i1; ++i) {
                double dot = 0.0;
                for (int64_t j = 0; j < l2; ++j) {
                    const int64_t idx = i * L2 + j;
                    dot += double(dprod(idx) * Cm[idx]) * R[idx];
                }
                const float d = float(dot);
                for (int64_t j = 0; j < l2; ++j) {
                    const int64_t idx = i * L2 + j;
                    GS[idx] += (dprod(idx) * Cm[idx] - d) * R[idx] * inv_t;
                }
            }
        });
        // column part: (d r - sum_i d r c) c / tau
        std::vector<double> cdot(static_cast<size_t>(l2), 0.0);
        for (int64_t i = 0; i < l1; ++i)
            for (int64_t j = 0; j < l2; ++j) {
                const int64_t idx = i * L2 + j;
                cdot[size_t(j)] += double(dprod(idx) * R[idx]) * Cm[idx];
            }
        double gt = 0.0;
        for (int64_t i = 0; i < l1; ++i)
            for (int64_t j = 0; j < l2; ++j) {
                const int64_t idx = i * L2 + j;
                GS[idx] += (dprod(idx) * R[idx] - float(cdot[size_t(j)])) * Cm[idx] * inv_t;
                gt -= double(GS[idx]) * S[idx] * inv_t;
            }
        grad_tau.data_ptr<float>()[b] = float(gt);
    });
    return {grad, grad_tau};
}

}  // namespace

TORCH_LIBRARY_IMPL(dot, CPU, m) {
    m.impl("sinkhorn", sinkhorn_cpu);
    m.impl("sinkhorn_log", sinkhorn_log_cpu);
    m.impl("sinkhorn_dual_forward", sinkhorn_dual_forward_cpu);
    m.impl("sinkhorn_spectral_preflight", spectral_preflight_cpu);
    m.impl("sinkhorn_with_grads_unrolled", with_grads_unrolled_cpu);
    m.impl("sinkhorn_with_grads_implicit", with_grads_implicit_cpu);
    m.impl("bidirectional_softmax", bidirectional_softmax_cpu);
    m.impl("bidirectional_softmax_backward", bidirectional_softmax_backward_cpu);
}
