/*
 * dot_amd — C ABI of the MI355X (gfx950) Sinkhorn and bidirectional-softmax engine.
 *
 * Plain pointers and sizes only.  Every pointer argument is device memory
 * owned by the caller (fp32 unless stated); the library allocates nothing on
 * its hot path: scratch comes from the caller's `workspace`, sized by the
 * matching *_workspace_bytes() query.  All work is enqueued on `stream`
 * (a hipStream_t); no call synchronises the device.  Functions return
 * DOT_OK (0) or a DOT_ERR_* code; dot_last_error() gives the message for the
 * calling thread.
 *
 * Layouts: matrices are row-major [B, M, N] (B batch elements, M rows, N
 * columns); row vectors are [B, M]; column vectors are [B, N].
 *
 * The reference implements this path as PyTorch custom ops whose CUDA
 * implementations call raw-pointer launchers.  Each entry point below replaces
 * the launchers named in its comment (paths relative to the reference root).
 */
#ifndef DOT_AMD_H
#define DOT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* dot_stream_t; /* same type as hipStream_t */

enum {
    DOT_OK = 0,
    DOT_ERR_INVALID_ARG = 1,  /* bad shape, pointer, size or parameter */
    DOT_ERR_WORKSPACE = 2,    /* workspace missing or smaller than the query */
    DOT_ERR_UNSUPPORTED = 3,  /* a shape this build does not handle (see message) */
    DOT_ERR_HIP = 4           /* a HIP launch or runtime call failed */
};

/* Flags of dot_sinkhorn_fwd_args.flags */
#define DOT_SK_RETURN_LOG 0x1    /* write log P instead of P (the reference's return_log) */
#define DOT_SK_KEEP_HISTORY 0x2  /* write u_t, v_t of every iteration for the unrolled backward */

/* Meaning of `scores` in the Sinkhorn calls. */
#define DOT_SCORES_LOG_ALPHA 1   /* scores are log_alpha; the log kernel is K = log_alpha / tau */
#define DOT_SCORES_COST (-1)     /* scores are a cost C; log_alpha = -C (dot/sinkhorn.py:1346) */

/* ---------------------------------------------------------------------- */
/* Sinkhorn forward                                                        */
/* ---------------------------------------------------------------------- */
typedef struct {
    const float* scores;   /* [B,M,N] log_alpha or cost, per scores_kind */
    const float* log_a;    /* [B,M] log row marginal, or NULL for -log(M) */
    const float* log_b;    /* [B,N] log column marginal, or NULL for -log(N) */
    int B, M, N;
    int scores_kind;       /* DOT_SCORES_LOG_ALPHA or DOT_SCORES_COST */
    float tau;             /* > 0 */
    int max_iter;          /* >= 0 */
    float tol;             /* > 0: stop after the first iteration with max|u_t - u_{t-1}| < tol
                              over the whole batch; <= 0: run max_iter iterations */
    int flags;             /* DOT_SK_* */
    float* plan;           /* [B,M,N] out: P (or log P); may be NULL */
    float* cost;           /* [B] out: sum(P * C) with C = -log_alpha; may be NULL */
    float* u_out;          /* [B,M] out: final row potential; may be NULL */
    float* v_out;          /* [B,N] out: final column potential; may be NULL */
    float* u_hist;         /* [max_iter,B,M] out when DOT_SK_KEEP_HISTORY */
    float* v_hist;         /* [max_iter,B,N] out when DOT_SK_KEEP_HISTORY */
    int32_t* iters_used;   /* device int32 out: iterations executed */
    int32_t* converged;    /* device int32 out: 1 if the tol test fired */
    void* workspace;
    size_t workspace_bytes;
    /* Optional exchange words of the register-resident kernels (see
     * dot_sinkhorn_exchange_bytes): NULL, and the library takes them from the
     * workspace and clears them with one more small kernel per call; or
     * caller-owned device memory of dot_sinkhorn_exchange_bytes() bytes,
     * zeroed once, used by calls on one stream only, with exchange_epoch
     * 1, 2, ... (at most DOT_SINKHORN_MAX_EPOCH) growing by one per call
     * (forward and backward calls share one sequence); zero the words again
     * before the sequence restarts at 1.  No counterpart in the reference. */
    void* exchange;
    uint32_t exchange_epoch;
} dot_sinkhorn_fwd_args;

/* Dual log-domain Sinkhorn: u_i = log a_i - LSE_j(K_ij + v_j), then
 * v_j = log b_j - LSE_i(K_ij + u_i), from u = v = 0, with the stopping test
 * evaluated on the device; P = safe_exp(K + u_i + v_j).
 * Replaces sinkhorn_dual_init_cuda / sinkhorn_dual_row_update_cuda /
 * sinkhorn_dual_col_update_cuda / sinkhorn_max_abs_diff_cuda /
 * sinkhorn_dual_materialize_cuda (src/sinkhorn/kernels.cuh:84-162) as driven by
 * sinkhorn_dual_vanilla_cuda (src/sinkhorn/torch_cuda.cpp:147-264), the
 * primal sinkhorn_forward_cuda (kernels.cuh:61) behind the sinkhorn /
 * sinkhorn_log ops (torch_cuda.cpp:599-715), and
 * sinkhorn_dual_forward_with_intermediates_cuda (kernels.cuh:164) when
 * DOT_SK_KEEP_HISTORY is set.  Ops: src/sinkhorn/registry.cpp:31-45.
 * Shapes beyond the one-launch tiers (batches larger than the chip holds,
 * rows longer than 4096 columns) run one launch pair per iteration; with
 * tol > 0 those calls read the device's stop test back after iterations 4, 8,
 * 16, ... (a wait on `stream` each, not while the stream is captured) and
 * stop launching once it has fired. */
/* For shapes that take the persistent streaming tier the workspace includes
 * room for a scaled copy of the kernel ([B,M,N] floats) that lets that tier
 * iterate without an exponential per element; a workspace of at least the
 * size without it (as the static scratch of dot_sinkhorn_forward_noalloc)
 * runs without it, to the same tolerance. */
size_t dot_sinkhorn_forward_workspace_bytes(int B, int M, int N, int max_iter, int flags);
int dot_sinkhorn_forward(const dot_sinkhorn_fwd_args* args, dot_stream_t stream);

/* Bytes of the static device scratch behind dot_sinkhorn_forward_noalloc. */
#define DOT_STATIC_SCRATCH_BYTES (64u << 20)

/* dot_sinkhorn_forward without a workspace argument and without any
 * allocation: args->workspace and args->workspace_bytes are ignored and the
 * scratch is a file-scope device array of DOT_STATIC_SCRATCH_BYTES per GPU,
 * held from the first call on that GPU until the process ends (the array is
 * a code object of its own, without kernels, which the HIP runtime's deferred
 * loading places on a GPU only when this call first looks it up there; using
 * the other entry points does not reserve it).  Shapes whose
 * workspace exceeds DOT_STATIC_SCRATCH_BYTES return DOT_ERR_UNSUPPORTED (the
 * workspace without the optional scaled kernel that
 * dot_sinkhorn_forward_workspace_bytes() adds for the persistent tier's
 * shapes; without it that tier iterates in the log domain throughout).
 * Results are those of dot_sinkhorn_forward.
 * All calls on one GPU share its array (each call clears what must start at
 * zero), so calls that overlap on one GPU — on different streams, or from
 * different threads — race and must be serialised by the caller.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). */
int dot_sinkhorn_forward_noalloc(const dot_sinkhorn_fwd_args* args, dot_stream_t stream);

/* Solver of dot_sinkhorn_method_args.method (the reference's method codes). */
#define DOT_SK_VANILLA 0
#define DOT_SK_MOMENTUM 1
#define DOT_SK_ANDERSON 2
#define DOT_SK_ADAM 3
/* Regularisation schedule of dot_sinkhorn_method_args.schedule. */
#define DOT_SK_SCHEDULE_NONE 0
#define DOT_SK_SCHEDULE_LINEAR 1
#define DOT_SK_SCHEDULE_EXPONENTIAL 2
#define DOT_SK_SCHEDULE_COSINE 3
#define DOT_SK_MAX_ANDERSON 64  /* longest Anderson ring this build holds: anderson_k above it
                                   is accepted while max_iter <= 64 (the ring never wraps) */

typedef struct {
    dot_sinkhorn_fwd_args base;  /* as for dot_sinkhorn_forward; DOT_SK_KEEP_HISTORY is not
                                    accepted (u_hist, v_hist unused) */
    int method;                  /* DOT_SK_VANILLA .. DOT_SK_ADAM */
    float omega;                 /* momentum over-relaxation */
    int anderson_k;              /* Anderson history >= 1; min(anderson_k, max_iter) <= DOT_SK_MAX_ANDERSON */
    float mixing_beta;           /* Anderson mixing */
    float lr, beta1, beta2, eps_adam;
    int bias_correction;         /* Adam: nonzero divides the moments by 1 - beta^t */
    float reg_start;             /* schedule start; <= 0 means 10 * tau */
    int schedule;                /* DOT_SK_SCHEDULE_* */
} dot_sinkhorn_method_args;

/* Accelerated and scheduled dual Sinkhorn: the reference's momentum (relaxed
 * u and v steps kept when the batch-wide max distance to the plain update
 * shrinks), Adam (moment-scaled steps, same acceptance test) and Anderson
 * (mixing of the last anderson_k (state, residual) pairs of x = (u, v), per
 * batch element) iterations, and the vanilla iteration under a linear,
 * exponential or cosine schedule of tau from reg_start to tau.  Every
 * acceptance and stopping decision is taken on the device.  With tol > 0 the
 * call waits on `stream` every 16 iterations to stop launching once the test
 * has fired (not while the stream is being captured).  The plan is
 * exp(K + u + v) at the target tau (the vanilla method: safe_exp).
 * Replaces sinkhorn_dual_forward_cuda_impl's method and schedule branches
 * (src/sinkhorn/torch_cuda.cpp:266-557: sinkhorn_dual_vanilla_cuda with a
 * schedule, :147-264; the method loop, :323-536; scheduled_tau_cuda, :61-84;
 * dual_fixed_point_map_cuda, :98-145) behind sinkhorn_dual_forward
 * (registry.cpp:31-36).  The reference's Anderson map hands a strided view of
 * v to a kernel that indexes it densely (torch_cuda.cpp:116-117 with
 * kernels.cu:518), so for B > 1 its iterates mix batch elements; this entry
 * point runs the per-element map (the two agree at B = 1). */
size_t dot_sinkhorn_forward_method_workspace_bytes(int B, int M, int N, int max_iter, int method,
                                                   int anderson_k);
int dot_sinkhorn_forward_method(const dot_sinkhorn_method_args* args, dot_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Sinkhorn backward                                                       */
/* ---------------------------------------------------------------------- */
/* L = sum(grad_plan * P) + grad_cost[b] * cost[b], cost = sum(P * C), with
 * C = scores for DOT_SCORES_COST and C = -scores for DOT_SCORES_LOG_ALPHA;
 * either term optional.  The plan's upstream gradient is G = grad_plan +
 * grad_cost[b] * C and, with g = the gradient through the plan w.r.t.
 * log_alpha:  DOT_SCORES_LOG_ALPHA: grad_scores = g - grad_cost[b] * P;
 * DOT_SCORES_COST: grad_scores = grad_cost[b] * P - g (the direct term of the
 * cost plus the path through the plan). */
typedef struct {
    const float* scores;      /* [B,M,N] */
    int scores_kind;
    const float* plan;        /* [B,M,N] P of the forward */
    const float* grad_plan;   /* [B,M,N] or NULL */
    const float* grad_cost;   /* [B] or NULL (with DOT_SK_GRAD_COST_SCALAR: one value for every element) */
    int B, M, N;
    float tau;
    int iters;                /* implicit: adjoint sweeps; unrolled: T (history length used) */
    const float* u_hist;      /* unrolled only: [T,B,M] */
    const float* v_hist;      /* unrolled only: [T,B,N] */
    float* grad_scores;       /* [B,M,N] out */
    float* grad_tau;          /* [B] out (per batch element) */
    void* workspace;
    size_t workspace_bytes;
    int32_t* status;          /* int32 out written by a kernel (device memory, or pinned host
                                 memory the device can reach), or NULL: 0 when the call's
                                 kernels finish normally, 1 when a cross-workgroup exchange
                                 timed out (the gradients are then NaN) */
    void* exchange;           /* optional exchange words, as in dot_sinkhorn_fwd_args */
    uint32_t exchange_epoch;
    int32_t* sweeps_used;     /* implicit only: [B] int32 out (device memory, or pinned host memory the
                                 device can reach), or NULL: adjoint sweeps executed per batch element */
    int flags;                /* DOT_SK_EXACT_SWEEPS, DOT_SK_GRAD_COST_SCALAR */
} dot_sinkhorn_bwd_args;

/* Flags of dot_sinkhorn_bwd_args.flags.  DOT_SK_EXACT_SWEEPS: run exactly
 * `iters` adjoint sweeps.  DOT_SK_GRAD_COST_SCALAR: grad_cost points to one
 * value that is every batch element's (the upstream gradient of cost.sum()),
 * so callers need not expand it to [B]. */
#define DOT_SK_EXACT_SWEEPS 0x4
#define DOT_SK_GRAD_COST_SCALAR 0x8

/* Implicit-function adjoint: up to `iters` Gauss-Seidel sweeps
 * lambda_i = (sum_k P G - sum_k P mu_k) / max(sum_k P, 1e-12),
 * mu_k = (sum_i P G - sum_i P lambda_i) / max(sum_i P, 1e-12),
 * grad = P (G - lambda_i - mu_k) / tau, grad_tau = -sum(grad * log_alpha) / tau.
 * Without DOT_SK_EXACT_SWEEPS, rows of at most 4096 columns (the register-
 * resident and persistent tiers, batches beyond the chip in slabs of them)
 * end a batch element's sweeps early once
 * they have converged, with d = max|mu_t - mu_{t-1}| and s the size of the
 * mu update's operands, max_k (|sum_i P G| + |sum_i P lambda|) / sum_i P:
 * when a sweep leaves mu unchanged (a fixed point: the result is the full
 * count's bit for bit); when three successive changes each shrank by at least
 * half and the geometric bound on everything the remaining sweeps could change
 * is at most 2^-22 s; or when d did not shrink, which exact arithmetic
 * excludes for a nonzero change (the sweeps have reached their fp32 rounding
 * floor), while at most 2^-18 s.  The
 * reference's GPU op runs every sweep (kernels.cu:1715-1718); its CPU op also
 * stops early, at a change below 1e-6 (kernels_cpu.cpp:276-312).  Other shapes
 * run every sweep.  sweeps_used reports what ran.
 * Replaces sinkhorn_backward_implicit_cuda (src/sinkhorn/kernels.cuh:325;
 * kernels.cu:1682-1726) behind sinkhorn_with_grads_implicit
 * (torch_cuda.cpp:803-871; registry.cpp:56). */
size_t dot_sinkhorn_backward_implicit_workspace_bytes(int B, int M, int N);
int dot_sinkhorn_backward_implicit(const dot_sinkhorn_bwd_args* args, dot_stream_t stream);

/* Reverse pass through the T recorded iterations with the reference's formula
 * (Gamma_Y = Gamma - exp(K+u_t+v_t) colsum(Gamma); Gamma = Gamma_Y -
 * exp(K+u_t+v_{t-1}) rowsum(Gamma_Y)); grad = Gamma / tau,
 * grad_tau = -sum(Gamma * log_alpha) / tau^2.
 * Replaces sinkhorn_backward_unrolled_dual_cuda (src/sinkhorn/kernels.cuh:292;
 * kernels.cu:1622-1680) behind sinkhorn_with_grads_unrolled
 * (torch_cuda.cpp:717-801; registry.cpp:52). */
size_t dot_sinkhorn_backward_unrolled_workspace_bytes(int B, int M, int N);
int dot_sinkhorn_backward_unrolled(const dot_sinkhorn_bwd_args* args, dot_stream_t stream);

typedef struct {
    const float* log_alpha;   /* [B,M,N] */
    int B, M, N;
    float tau;                /* > 0 */
    int n_power;              /* power iterations, >= 1 */
    float* tau_est;           /* [B] out: contraction estimate in [0, 0.999999] */
    void* workspace;
    size_t workspace_bytes;
} dot_spectral_preflight_args;

/* Spectral contraction estimate behind n_iters='auto': with
 * P = softmax_row(log_alpha / tau), n_power deflated power iterations
 * u = centre(P v), v = centre_normalise(P^T u) from the reference's
 * deterministic sin() start vector, then tau_est = ||centre(P v)||.
 * Replaces sinkhorn_spectral_preflight_cuda (src/sinkhorn/kernels.cuh;
 * kernels.cu:141-241, :1509-1532) behind sinkhorn_spectral_preflight
 * (torch_cuda.cpp:559-593; registry.cpp:48). */
size_t dot_sinkhorn_spectral_preflight_workspace_bytes(int B, int M, int N);
int dot_sinkhorn_spectral_preflight(const dot_spectral_preflight_args* args, dot_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Bidirectional softmax                                                   */
/* ---------------------------------------------------------------------- */
typedef struct {
    const float* sim;         /* [B,L1,L2] */
    const int32_t* lengths;   /* [B,2] valid (rows, cols) per batch element, device int32;
                                 NULL: every element is full (L1, L2) */
    int B, L1, L2;
    float tau;
    float* out;               /* [B,L1,L2] sqrt(1e-9 + r*c) in the valid region, else 0 */
    float* row_sm;            /* [B,L1,L2] row softmax r, or NULL */
    float* col_sm;            /* [B,L1,L2] column softmax c, or NULL */
    /* Statistics, with y2 = sim * (1/tau) * log2(e): the max plane holds max y2
     * over the row (column), the sum plane sum exp2(y2 - max) (the softmax
     * denominator).  Only the backward of this library reads them back. */
    float* row_stats;         /* [B,2,L1] row max plane then row sum plane, or NULL */
    float* col_stats;         /* [B,2,L2] column max plane then column sum plane, or NULL */
    void* workspace;
    size_t workspace_bytes;
    /* Optional exchange words of the one-pass kernels (both L1 and L2 in
     * 513..1024, B at least the GPU's XCD count, row_sm and col_sm NULL; see
     * dot_bidisoftmax_exchange_bytes): NULL, and the library takes them from
     * the workspace and clears them with one more small kernel per call; or
     * caller-owned device memory of dot_bidisoftmax_exchange_bytes() bytes,
     * zeroed once, used by calls on one stream only, with exchange_epoch
     * 1, 2, ... (at most DOT_BIDISOFTMAX_MAX_EPOCH) growing by one per call
     * (forward and backward calls share one sequence); zero the words again
     * before the sequence restarts at 1.  No counterpart in the reference. */
    void* exchange;
    uint32_t exchange_epoch;
} dot_bidisoftmax_fwd_args;

/* Replaces bidirectional_softmax_forward_cuda
 * (src/bidirectional_softmax/kernels.cuh:27; kernels.cu:417-448) behind the
 * bidirectional_softmax op (bidirectional_softmax/torch_cuda.cpp:42-76;
 * registry.cpp:31).  Runs on `stream` with no device synchronisation. */
size_t dot_bidisoftmax_forward_workspace_bytes(int B, int L1, int L2);
int dot_bidisoftmax_forward(const dot_bidisoftmax_fwd_args* args, dot_stream_t stream);

typedef struct {
    const float* sim;         /* [B,L1,L2] */
    const int32_t* lengths;   /* [B,2] */
    int B, L1, L2;
    float tau;
    const float* grad_out;    /* [B,L1,L2] */
    /* Either the forward's buffers (out, row_sm, col_sm all non-NULL) ... */
    const float* out;
    const float* row_sm;
    const float* col_sm;
    /* ... or its statistics, from which r, c and out are recomputed from sim. */
    const float* row_stats;   /* [B,2,L1] as written by the forward */
    const float* col_stats;   /* [B,2,L2] */
    float* grad_sim;          /* [B,L1,L2] out (0 outside the valid region) */
    float* grad_tau;          /* [B] out: -sum(grad_sim * sim) / tau over the valid region,
                                 or NULL to skip it (the autograd path has no tau gradient) */
    void* workspace;
    size_t workspace_bytes;
    /* As in dot_bidisoftmax_fwd_args (the one-pass backward runs from the
     * statistics, with grad_tau NULL). */
    void* exchange;
    uint32_t exchange_epoch;
} dot_bidisoftmax_bwd_args;

/* Replaces bidirectional_softmax_backward_cuda
 * (src/bidirectional_softmax/kernels.cuh:56; kernels.cu:450-501) behind the
 * bidirectional_softmax_backward op (bidirectional_softmax/torch_cuda.cpp:78-139;
 * registry.cpp:34). */
size_t dot_bidisoftmax_backward_workspace_bytes(int B, int L1, int L2);
int dot_bidisoftmax_backward(const dot_bidisoftmax_bwd_args* args, dot_stream_t stream);

/* Size of the caller-owned exchange words (the `exchange` fields above) and
 * the largest call epoch they take.  No counterpart in the reference. */
#define DOT_BIDISOFTMAX_MAX_EPOCH 1048575u
size_t dot_bidisoftmax_exchange_bytes(void);

/* Size of the caller-owned exchange words of the Sinkhorn calls (the
 * `exchange` fields of dot_sinkhorn_fwd_args and dot_sinkhorn_bwd_args) for
 * the current device, and the largest call epoch they take.  Calls whose
 * iteration count (max_iter, iters) exceeds DOT_SINKHORN_MAX_TAGGED_ITERS use
 * the workspace instead.  No counterpart in the reference. */
#define DOT_SINKHORN_MAX_EPOCH 65534u
#define DOT_SINKHORN_MAX_TAGGED_ITERS 65533
size_t dot_sinkhorn_exchange_bytes(void);

/* ---------------------------------------------------------------------- */
/* Diagnostics (no counterpart in the reference)                           */
/* ---------------------------------------------------------------------- */
/* Message of the calling thread's most recent failure ("" after success). */
const char* dot_last_error(void);
/* Library version string. */
const char* dot_version(void);

/* Kernel-duration profiler: when enabled, every launch is bracketed by two
 * HIP events on its stream.  dot_profile_collect() waits for the recorded
 * events and folds them into per-kernel totals; dot_profile_query() reads a
 * total by kernel name.  For measurement only: it adds event records between
 * launches. */
void dot_profile_enable(int on);
/* Restrict the profiler to a comma-separated list of kernel names (NULL or
 * "" selects every kernel). */
void dot_profile_select(const char* names);
int dot_profile_collect(void);
int dot_profile_query(const char* kernel, int64_t* launches, double* total_ms);
void dot_profile_reset(void);
/* Disable the profiler, wait for its recorded events and destroy every event
 * it holds.  Call before the process exits if the profiler was ever enabled:
 * events left to process teardown outlive the HIP runtime. */
int dot_profile_shutdown(void);

#ifdef __cplusplus
}
#endif

#endif /* DOT_AMD_H */
