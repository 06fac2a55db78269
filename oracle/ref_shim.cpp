// TEST INFRASTRUCTURE ONLY — never linked into the product.
//
// extern "C" entry points over the reference's own torch-free CPU kernels, so
// that Python tests can call them through ctypes.  The kernels themselves are
// compiled from their original location under /root/reference/src by
// oracle/Makefile; nothing of the reference is copied into this repository.
//
// Wrapped functions (signatures from the reference headers):
//   dot::sinkhorn::sinkhorn_forward_cpu                      src/sinkhorn/kernels_cpu.h:29
//   dot::sinkhorn::sinkhorn_forward_with_intermediates_cpu   src/sinkhorn/kernels_cpu.h:53
//   dot::sinkhorn::sinkhorn_backward_unrolled_cpu            src/sinkhorn/kernels_cpu.h:81
//   dot::sinkhorn::sinkhorn_backward_implicit_cpu            src/sinkhorn/kernels_cpu.h:111
//   dot::bidirectional_softmax::bidirectional_softmax_forward_cpu   src/bidirectional_softmax/kernels_cpu.h:14
//   dot::bidirectional_softmax::bidirectional_softmax_backward_cpu  src/bidirectional_softmax/kernels_cpu.h:27

#include "sinkhorn/kernels_cpu.h"
#include "bidirectional_softmax/kernels_cpu.h"

extern "C" {

void ref_sinkhorn_forward(const float* log_alpha, float* out, const float* log_a,
                          const float* log_b, int B, int n, int m, float tau,
                          int n_iters, int return_log) {
    dot::sinkhorn::sinkhorn_forward_cpu(log_alpha, out, log_a, log_b, B, n, m, tau,
                                        n_iters, return_log != 0);
}

void ref_sinkhorn_forward_with_intermediates(const float* log_alpha, float* P, float* log_X,
                                             float* log_Y, const float* log_a,
                                             const float* log_b, int B, int n, int m,
                                             float tau, int n_iters) {
    dot::sinkhorn::sinkhorn_forward_with_intermediates_cpu(log_alpha, P, log_X, log_Y, log_a,
                                                           log_b, B, n, m, tau, n_iters);
}

void ref_sinkhorn_backward_unrolled(const float* log_alpha, const float* P, const float* grad_P,
                                    const float* log_X, const float* log_Y, const float* log_a,
                                    const float* log_b, float* grad_log_alpha, float* grad_tau,
                                    int B, int n, int m, float tau, int n_iters) {
    dot::sinkhorn::sinkhorn_backward_unrolled_cpu(log_alpha, P, grad_P, log_X, log_Y, log_a,
                                                  log_b, grad_log_alpha, grad_tau, B, n, m,
                                                  tau, n_iters);
}

void ref_sinkhorn_backward_implicit(const float* log_alpha, const float* P, const float* grad_P,
                                    const float* log_a, const float* log_b,
                                    float* grad_log_alpha, float* grad_tau, int B, int n, int m,
                                    float tau, int max_iters, float tol) {
    dot::sinkhorn::sinkhorn_backward_implicit_cpu(log_alpha, P, grad_P, log_a, log_b,
                                                  grad_log_alpha, grad_tau, B, n, m, tau,
                                                  max_iters, tol);
}

void ref_bidi_forward(const float* sim, float* out, float* row_sm, float* col_sm,
                      const int* lengths, int B, int L1, int L2, float T) {
    dot::bidirectional_softmax::bidirectional_softmax_forward_cpu(sim, out, row_sm, col_sm,
                                                                  lengths, B, L1, L2, T);
}

void ref_bidi_backward(const float* sim, const float* out, const float* grad_out,
                       const float* row_sm, const float* col_sm, float* grad_sim,
                       float* grad_T, const int* lengths, int B, int L1, int L2, float T) {
    dot::bidirectional_softmax::bidirectional_softmax_backward_cpu(
        sim, out, grad_out, row_sm, col_sm, grad_sim, grad_T, lengths, B, L1, L2, T);
}

}  // extern "C"
