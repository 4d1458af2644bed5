/*
 * tgbwd.h — C-ABI of libtgbwd.so, the gfx950 backward-pass engine behind the
 * tensor_gpu_v2 API (DragonShadows1978/Project-Tensor).
 *
 * Conventions
 *  - Every function returns int: 0 on success, negative on error
 *    (-1 invalid argument, -2 HIP error, -3 unsupported, -4 workspace too small);
 *    tg_last_error() returns the thread's last message.
 *  - Pointers are device pointers unless stated; the caller owns every buffer,
 *    the library keeps no reference after return.
 *  - `stream` is a hipStream_t (NULL = default stream).  Work is asynchronous
 *    on that stream; only tg_stream_sync waits.
 *  - dtype codes: 0 = fp32, 1 = fp16, 2 = bf16, 3 = fp64.  fp64 (float64 data,
 *    which the reference keeps in float64, _core.py:173-193) is computed in double by
 *    the activations, tg_axpby(z), tg_fill, softmax, LayerNorm, tg_reduce_rows,
 *    tg_broadcast_mul_sum, tg_gemm (dtype_ab = dtype_c = 3), GradScaler unscale and
 *    clipping, and by tg_axpbyz64, tg_cross_entropy_*_f64 and tg_adam_step_f64 (double
 *    scalars); BatchNorm, embedding, FlashAttention and the transpose-add reject code 3.
 *  - `accumulate` != 0 means out += result (the reference's `grad += local`
 *    closures); 0 means out = result (out is not read).
 *  - Tensors are contiguous row-major unless leading dimensions are passed.
 *  - Element counts and offsets are 64-bit throughout; an elementwise call whose
 *    launch would exceed the 2^32 work-items of one dispatch (the activations and
 *    tg_unary_bwd: more than 2^32 16-byte vectors, i.e. 2^35 fp16 or 2^34 fp32
 *    elements) returns -1 instead of launching.
 *
 * Each entry cites the reference code it replaces (paths are relative to the
 * reference repository root).
 */
#ifndef TGBWD_H
#define TGBWD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime ---------------------------------------------------------- */
/* Select `device` and check that it is gfx950.  Replaces the implicit CuPy
 * device context (tensor_gpu_v2/_core.py:16, :116-125). */
int tg_init(int device);
const char* tg_last_error(void);
int tg_version(void);
int tg_stream_sync(void* stream);

/* ---- elementwise activations ------------------------------------------ */
/* dx (+)= dy * gelu'(x), tanh approximation.
 * Replaces RawKernel gelu_backward(x, grad_out, grad_in, n) and the
 * `self.grad += grad_in` that follows it (_core.py:493-507, :1185-1190),
 * and the xp fallback (_core.py:1199-1206). */
int tg_gelu_bwd(int dtype, const void* x, const void* dy, void* dx, int64_t n, int accumulate,
                void* stream);
/* dx (+)= dy * silu'(x).  Replaces silu_backward (_core.py:522-533, :1225-1230)
 * and the xp path (_core.py:1237-1243). */
int tg_silu_bwd(int dtype, const void* x, const void* dy, void* dx, int64_t n, int accumulate,
                void* stream);
/* dx (+)= f'(a) * dy for the other pointwise ops, in the reference closure's order
 * (float/double data in their own precision, fp16/bf16 in fp32 rounded once).
 * op: 0 ReLU, a = y: (y > 0) * dy             (_core.py:1149-1157)
 *     1 LeakyReLU, a = x: (x >= 0 ? 1 : param) * dy (_core.py:1159-1170)
 *     2 sigmoid, a = y: y * (1 - y) * dy       (_core.py:1262-1272)
 *     3 tanh, a = y: (1 - y*y) * dy            (_core.py:1274-1282)
 *     4 exp, a = y: y * dy
 *     5 log, a = x: dy / x
 *     6 power x ** param, a = x: (param * x ** (param - 1)) * dy (_core.py:973-981;
 *       a / b runs as a * b ** -1, _core.py:993-995); x ** e uses 1, sqrt, x, x*x and
 *       1/x for e = 0, 0.5, 1, 2, -1 as NumPy's power does, pow otherwise
 *     7 Swish x * sigmoid(param * x), a = x: (s + param*x*s*(1 - s)) * dy with
 *       s = 1 / (1 + exp(-param*x))               (_core.py:1248-1260) */
int tg_unary_bwd(int dtype, int op, const void* a, const void* dy, void* dx, int64_t n,
                 double param, int accumulate, void* stream);
/* log_softmax backward over the last axis of [rows, cols]:
 * dx (+)= dy - exp(y) * sum_row(dy) (_core.py:1301-1314). */
int tg_log_softmax_bwd(int dtype, const void* y, const void* dy, void* dx, int64_t rows,
                       int64_t cols, int accumulate, void* stream);
/* max backward with x viewed as [rows, cols] (reduced axes last), r [rows] the
 * maxima, g [rows] their upstream gradient: dx (+)= (x == r) * g / count(x == r) per
 * row (_core.py:1115-1132; min is -max(-x), :1134-1135). */
int tg_max_bwd(int dtype, const void* x, const void* r, const void* g, void* dx, int64_t rows,
               int64_t cols, int accumulate, void* stream);
/* Scatter-add of an integer-array / mask __getitem__ (_core.py:918-929, whose
 * _scatter_add is NumPy's add.at on the CPU path, :890-916): for each of nseg
 * distinct flat indices target[s], grad[target[s]] += (sum of src[order[j]] for j in
 * [start[s], start[s+1]), added in j order with the dtype's rounding at every step).
 * order is a stable sort of the selected elements by flat index (int64 [n]), start
 * is int64 [nseg + 1], src holds the upstream gradient of the selected elements
 * (contiguous, grad's dtype).  Deterministic: one thread owns each target. */
int tg_index_add_sorted(int dtype, void* grad, int64_t nseg, const int64_t* target,
                        const int64_t* start, const int64_t* order, const void* src,
                        void* stream);
/* Forward kernels feeding the above: gelu_forward (_core.py:479-491),
 * silu_forward (_core.py:510-520). */
int tg_gelu_fwd(int dtype, const void* x, void* y, int64_t n, void* stream);
int tg_silu_fwd(int dtype, const void* x, void* y, int64_t n, void* stream);
/* y = alpha*x + beta*y (beta == 0: y not read), x/y dtypes may differ.
 * The generic `parent.grad += g` accumulation of the closures (_core.py:945-966). */
int tg_axpby(int dtype_x, const void* x, int dtype_y, void* y, int64_t n, float alpha,
             float beta, void* stream);
/* z = alpha*x + beta*y with z of y's dtype (z may equal y).  The out-of-place form of
 * the same accumulation, used when the gradient buffer being added to is shared with
 * another node (copy-on-write; the reference's `+=` creates a new array there too,
 * _core.py:945-966). */
int tg_axpbyz(int dtype_x, const void* x, int dtype_y, const void* y, void* z, int64_t n,
              float alpha, float beta, void* stream);
/* tg_axpbyz with double scalars, for fp64 operands (x or y fp64, the other fp64 or fp32;
 * arithmetic in double, z of y's dtype).  No reference counterpart of its own: it keeps
 * scale factors such as 1/n of a mean exact to double for float64 gradients. */
int tg_axpbyz64(int dtype_x, const void* x, int dtype_y, const void* y, void* z, int64_t n,
                double alpha, double beta, void* stream);
/* Fill with a constant by a kernel (grad zeroing; graph-capture safe). */
int tg_fill(int dtype, void* y, int64_t n, float value, void* stream);

/* ---- row-wise ----------------------------------------------------------- */
/* Softmax over the last axis of a [rows, cols] matrix (_core.py:1286-1292). */
int tg_softmax_fwd(int dtype, const void* x, void* y, int64_t rows, int64_t cols, void* stream);
/* dx (+)= y * (dy - rowsum(dy*y))  (_core.py:1294-1297). */
int tg_softmax_bwd(int dtype, const void* y, const void* dy, void* dx, int64_t rows,
                   int64_t cols, int accumulate, void* stream);
/* LayerNorm forward over the last axis; saves mean and rstd = 1/sqrt(var+eps)
 * per row (fp32).  gamma/beta fp32.  (_nn.py:900-919)  dtype 3 (fp64 x, y, dy, dx): mean
 * and rstd point to double arrays; gamma/beta and dgamma/dbeta stay fp32 (the
 * reference's module parameters are float32, _nn.py:896-897). */
int tg_layernorm_fwd(int dtype, const void* x, const float* gamma, const float* beta, void* y,
                     float* mean, float* rstd, int64_t rows, int64_t cols, float eps,
                     void* stream);
/* LayerNorm backward (_nn.py:921-942): dx (+)= rstd*(g - mean(g) - xhat*mean(g*xhat)),
 * g = dy*gamma, xhat = (x-mean)*rstd; dgamma (+)= sum dy*xhat, dbeta (+)= sum dy
 * (either may be NULL).  Workspace from tg_layernorm_bwd_workspace. */
size_t tg_layernorm_bwd_workspace(int dtype, int64_t rows, int64_t cols);
int tg_layernorm_bwd(int dtype, const void* x, const float* mean, const float* rstd,
                     const float* gamma, const void* dy, void* dx, float* dgamma, float* dbeta,
                     int64_t rows, int64_t cols, int accumulate_dx, int accumulate_params,
                     void* workspace, size_t workspace_bytes, void* stream);
/* tg_layernorm_bwd writing dx = (LayerNorm dx) + dx_add, where dx_add may be another
 * buffer than dx: the input's gradient is shared with another node (the residual
 * add's pass-through, _core.py:941-968, then the LayerNorm closure's parent.grad +=),
 * so the sum goes to the input's own new buffer in the same pass, with no copy first.
 * dx_add == dx is tg_layernorm_bwd with accumulate_dx. */
int tg_layernorm_bwd_add(int dtype, const void* x, const float* mean, const float* rstd,
                         const float* gamma, const void* dy, const void* dx_add, void* dx,
                         float* dgamma, float* dbeta, int64_t rows, int64_t cols,
                         int accumulate_params, void* workspace, size_t workspace_bytes,
                         void* stream);
/* With dgamma and dbeta both NULL, tg_layernorm_bwd(_add) leaves the dgamma and dbeta
 * partials in the workspace's first 2*K*cols floats (K rows each, dgamma's first) for a
 * later finish; tg_layernorm_bwd_partials gives K for that call's shape and pointers,
 * or -1 where the partials cannot be finished by tg_sum_partials2_group (fp64, or a
 * partial count it does not cover).  During Tensor.backward() the LayerNorm closures
 * (_nn.py:921-942) leave their partials this way and the parameter gradients are
 * finished together when the sweep ends. */
int64_t tg_layernorm_bwd_partials(int dtype, const void* x, const void* dy, const void* dx,
                                  const void* dx_add, int64_t rows, int64_t cols);
/* n finishes in one launch: out0[i] (+)= column sums of parts[i][0:K[i]][0:cols[i]] and
 * out1[i] (+)= those of parts[i][K[i]:2K[i]] (fp32; acc[i] non-zero: add to the
 * outputs; acc NULL: overwrite), each equal to finishing member i on its own.  Host
 * arrays of n entries; an output may be NULL (skipped). */
int tg_sum_partials2_group(int n, const float* const* parts, const int64_t* K,
                           const int64_t* cols, float* const* out0, float* const* out1,
                           const int* acc, void* stream);
/* tg_layernorm_bwd without a workspace argument and without any allocation: the
 * partial sums live in a fixed device array of the library (one per GPU, held until
 * the process ends; tg_layernorm_bwd_noalloc_max_scratch() bytes).  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops).  Shapes whose partials exceed the scratch
 * return -1 with a message.  Calls that overlap on one GPU share the scratch and race:
 * calls on one stream are ordered by it; callers using several streams order their
 * calls themselves (an event, as under graph capture, where a library-side wait on
 * another stream's event is not allowed). */
size_t tg_layernorm_bwd_noalloc_max_scratch(void);
int tg_layernorm_bwd_noalloc(int dtype, const void* x, const float* mean, const float* rstd,
                             const float* gamma, const void* dy, void* dx, float* dgamma,
                             float* dbeta, int64_t rows, int64_t cols, int accumulate_dx,
                             int accumulate_params, void* stream);
/* Strided broadcast multiply with reduction over one ndim-dimensional index space:
 *   out[o(i)] (+)= alpha * sum_i a[a(i)] * b[b(i)]
 * with element strides per dimension (input stride 0 = broadcast, output stride 0 =
 * summed away); b may be NULL (taken as 1); dtypes 0-3 (fp32, fp16, bf16, fp64) in any
 * mix.  Replaces Tensor._unbroadcast (_core.py:1380-1424), the __mul__ backward
 * (_core.py:955-968: other * grad, unbroadcast) and the sum/mean backward broadcast
 * (_core.py:1078-1087), and strided copies/casts of gradient buffers.  Deterministic
 * (fixed summation order, fp32 or fp64 accumulation). */
int tg_broadcast_mul_sum(int ndim, const int64_t* shape, int dtype_a, const void* a,
                         const int64_t* strides_a, int dtype_b, const void* b,
                         const int64_t* strides_b, int dtype_out, void* out,
                         const int64_t* strides_out, double alpha, int accumulate,
                         void* stream);
/* out[c] (+)= sum_r in[r][c]: Tensor._unbroadcast's leading-dimension sums
 * (_core.py:1380-1424), e.g. the Linear bias gradient.  fp64 input or output: summed in
 * double, in fixed order. */
size_t tg_reduce_rows_workspace(int64_t rows, int64_t cols);
int tg_reduce_rows(int dtype_in, const void* in, int dtype_out, void* out, int64_t rows,
                   int64_t cols, int accumulate, void* workspace, size_t workspace_bytes,
                   void* stream);

/* ---- batch norm (+ReLU), fp32 (fp64 forms below) ------------------------- */
/* layout: 0 = NHWC ([N*H*W, C]), 1 = NCHW.  HW = H*W. */
size_t tg_batchnorm_workspace(int layout, int64_t N, int64_t C, int64_t HW);
/* Training forward of FusedBatchNormReLU / BatchNorm2D (_nn.py:794-810, :701-714):
 * batch mean/var (population), rstd, running-stat EMA (either running pointer
 * may be NULL), y = [relu](gamma*xhat + beta).  var may be NULL. */
int tg_batchnorm_fwd_train(int layout, const float* x, const float* gamma, const float* beta,
                           float* y, float* mean, float* rstd, float* var, float* running_mean,
                           float* running_var, float momentum, int64_t N, int64_t C, int64_t HW,
                           float eps, int relu, void* workspace, size_t workspace_bytes,
                           void* stream);
/* Training backward (_nn.py:812-833; BatchNorm2D _nn.py:720-736 with relu = 0):
 * dx (+)= gamma*rstd*(dy_m - mean(dy_m) - xhat*mean(dy_m*xhat)), dy_m = dy*[out>0],
 * dgamma (+)= sum dy_m*xhat, dbeta (+)= sum dy_m (either may be NULL). */
int tg_batchnorm_bwd(int layout, const float* x, const float* mean, const float* rstd,
                     const float* gamma, const float* beta, const float* dy, float* dx,
                     float* dgamma, float* dbeta, int64_t N, int64_t C, int64_t HW, int relu,
                     int accumulate_dx, int accumulate_params, void* workspace,
                     size_t workspace_bytes, void* stream);
/* Training forward on float64 data (_nn.py:794-810 on float64 arrays): batch mean/var
 * (two passes), rstd, the running EMA in double (either running pointer may be NULL),
 * y = [relu](gamma*xhat + beta) in double; gamma/beta are the fp32 parameters. */
int tg_batchnorm_fwd_train_f64(int layout, const double* x, const float* gamma,
                               const float* beta, double* y, double* mean, double* rstd,
                               double* var, double* running_mean, double* running_var,
                               double momentum, int64_t N, int64_t C, int64_t HW, double eps,
                               int relu, void* stream);
/* Backward with the reference's own formula against given per-channel statistics
 * (mean, rstd in double): dout = dy*[out > 0], dgamma (+)= sum dout*xhat, dbeta (+)=
 * sum dout, dx (+)= dout*gamma*rstd + dvar*(2/m)*xc + dmean/m with
 * dvar = -0.5*rstd^3*sum(dout*gamma*xc), dmean = -rstd*sum(dout*gamma) +
 * dvar*(-2/m)*sum(xc) (_nn.py:812-833, :720-736).  Serves float64 data (dtype 3) and
 * the eval-mode BatchNorm2D backward on the running statistics (dtype 0 or 3), where
 * sum(xc) != 0.  Sums in double; the fp32 parameter gradients are rounded once.
 * Workspace: tg_batchnorm_stats_workspace(C) bytes. */
size_t tg_batchnorm_stats_workspace(int64_t C);
int tg_batchnorm_bwd_stats(int dtype, int layout, const void* x, const double* mean,
                           const double* rstd, const float* gamma, const float* beta,
                           const void* dy, void* dx, float* dgamma, float* dbeta, int64_t N,
                           int64_t C, int64_t HW, int relu, int accumulate_dx,
                           int accumulate_params, void* workspace, size_t workspace_bytes,
                           void* stream);

/* ---- optimizers and gradient hygiene (multi-tensor, host pointer lists) --- */
/* Adam / AdamW step over `ntensors` fp32 tensors (_nn.py:1413-1442, FusedAdam
 * fused_adam_step _training.py:2198-2220, launch _training.py:2250-2268):
 * decoupled decay p -= lr*wd*p first, then the moment updates and
 * p -= lr*(m/bc1)/(sqrt(v/bc2)+eps).  max_exp_avg_sq != NULL selects AMSGrad
 * (_nn.py:1436-1438).  Hyper-parameters are doubles (Python floats in the
 * reference) combined in double and rounded once to fp32. */
int tg_adam_step(int ntensors, float* const* params, const float* const* grads,
                 float* const* exp_avg, float* const* exp_avg_sq, float* const* max_exp_avg_sq,
                 const int64_t* numel, double lr, double beta1, double beta2, double eps,
                 double weight_decay, double bias_correction1, double bias_correction2,
                 void* stream);
/* tg_adam_step that also writes each updated parameter, rounded to lowp_dtype (fp16
 * or bf16 code), to lowp[i] where lowp[i] != NULL.  Replaces the per-forward weight
 * cast of autocast (_core.py:185-191 casts every fp32 parameter to fp16 when the
 * forward reads it): the copy is produced in the optimizer pass that changes the
 * weights, so the next forward finds it current.  No reference counterpart of its
 * own; results of the update are those of tg_adam_step. */
int tg_adam_step_lowp(int ntensors, float* const* params, const float* const* grads,
                      float* const* exp_avg, float* const* exp_avg_sq,
                      float* const* max_exp_avg_sq, const int64_t* numel, double lr,
                      double beta1, double beta2, double eps, double weight_decay,
                      double bias_correction1, double bias_correction2, int lowp_dtype,
                      void* const* lowp, void* stream);
/* tg_adam_step / tg_adam_step_lowp (lowp NULL: no copies) reading each gradient as
 * (g * grad_mul1) * grad_mul2 in fp32: the values an in-place unscale by grad_mul1
 * (GradScaler.unscale_, _nn.py:1795-1833) followed by an in-place clip scaling by
 * grad_mul2 (clip_grad_norm_, _nn.py:1620-1624) would leave, so the gradients can stay
 * loss-scaled in memory until the optimizer reads them.  No reference counterpart of its
 * own; the update is tg_adam_step's. */
int tg_adam_step_scaled(int ntensors, float* const* params, const float* const* grads,
                        float* const* exp_avg, float* const* exp_avg_sq,
                        float* const* max_exp_avg_sq, const int64_t* numel, double lr,
                        double beta1, double beta2, double eps, double weight_decay,
                        double bias_correction1, double bias_correction2, float grad_mul1,
                        float grad_mul2, int lowp_dtype, void* const* lowp, void* stream);
/* GradScaler.unscale_ (_nn.py:1795-1833): g *= mul (if write); flags[i] (device,
 * cleared first) |= 1 if tensor i had a non-finite value, |= 2 if the scaled
 * tensor has one. */
int tg_unscale_check(int ntensors, int dtype, void* const* grads, const int64_t* numel, float mul,
                     int write, int* flags, void* stream);
/* GradScaler.unscale_ with zero_nan_grads (_nn.py:1816-1829): every gradient i whose
 * device flag flags[i] (from tg_unscale_check) is non-zero is zeroed whole, decided on
 * the device, so the flags need no read-back before the next kernels. */
int tg_zero_flagged(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                    const int* flags, void* stream);
/* clip_grad_norm_ (_nn.py:1563-1626) reduction: out[0] (device double) =
 * sum g^2 (kind 0), max|g| (kind 1) or sum |g|^p (kind 2) over finite entries;
 * flags[i] |= 1 when tensor i has non-finite entries. */
size_t tg_grad_norm_workspace(int ntensors, const int64_t* numel);
int tg_grad_norm(int ntensors, int dtype, void* const* grads, const int64_t* numel, int norm_kind,
                 float p, double* out, int* flags, void* workspace, size_t workspace_bytes,
                 void* stream);
/* GradScaler.unscale_ (_nn.py:1795-1833) and clip_grad_norm_'s L2 reduction
 * (_nn.py:1588-1612) in one read-only pass: flags[i] as tg_unscale_check's, and out[0]
 * (device double) = the sum of squares the gradients would have after
 * tg_unscale_check(mul, write = 1) and tg_zero_flagged, bit for bit (tg_grad_norm's
 * chunks and order; a flagged tensor counts zero).  fp32, fp16 and bf16 gradients.
 * Workspace: tg_unscale_norm_workspace(ntensors, numel) bytes. */
size_t tg_unscale_norm_workspace(int ntensors, const int64_t* numel);
int tg_unscale_norm(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                    float mul, int* flags, double* out, void* workspace,
                    size_t workspace_bytes, void* stream);
/* xp.where(isfinite(g), g, 0) per tensor (_nn.py:1596). */
int tg_zero_nonfinite(int ntensors, int dtype, void* const* grads, const int64_t* numel,
                      void* stream);
/* tg_adam_step for float64 parameters, gradients and moments, in double throughout
 * (the reference's Adam on float64 arrays, _nn.py:1413-1442). */
int tg_adam_step_f64(int ntensors, double* const* params, const double* const* grads,
                     double* const* exp_avg, double* const* exp_avg_sq,
                     double* const* max_exp_avg_sq, const int64_t* numel, double lr,
                     double beta1, double beta2, double eps, double weight_decay,
                     double bias_correction1, double bias_correction2, void* stream);

/* ---- dense contractions (MFMA) ------------------------------------------ */
/* Batched row-major GEMM: C[b] = alpha * op(A[b]) @ op(B[b]) + beta * C[b],
 * op(A) is [M,K] (trans_a = 0: A[m*lda+k]; 1: A[k*lda+m]), op(B) is [K,N]
 * (trans_b = 0: B[k*ldb+n]; 1: B[n*ldb+k]); stride 0 broadcasts an operand.
 * dtype_ab in {fp32, fp16, bf16}; dtype_c is fp32 or dtype_ab; or dtype_ab = dtype_c =
 * fp64 (fp64 matrix cores, v_mfma_f64_16x16x4f64).  Serves the
 * matmul forward and its backward dA = dC @ B^T, dB = A^T @ dC
 * (_core.py:999-1068). */
int tg_gemm(int dtype_ab, int dtype_c, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
            float alpha, const void* A, int64_t lda, int64_t stride_a, const void* B,
            int64_t ldb, int64_t stride_b, float beta, void* C, int64_t ldc, int64_t stride_c,
            int64_t batch, void* stream);
/* C = alpha*op(A)@op(B) + bias[n] (fp32 bias of length N, added in the epilogue before
 * the rounding to dtype_c): the Linear forward y = x @ w + b (_nn.py:258-285, the
 * matmul then the broadcast add of _core.py:941-968) as one GEMM. */
int tg_gemm_bias(int dtype_ab, int dtype_c, int trans_a, int trans_b, int64_t M, int64_t N,
                 int64_t K, float alpha, const void* A, int64_t lda, const void* B, int64_t ldb,
                 const float* bias, void* C, int64_t ldc, void* stream);

/* Weight and bias gradients of a Linear layer y = x @ w + b from one pass over the
 * output gradient (the matmul node's dB = A^T @ dC, _core.py:1064-1068, and the
 * broadcast-add node's unbroadcast sum of _core.py:1380-1424, as Linear.__call__ builds
 * them, _nn.py:258-285): dW[M,N] (+)= X^T @ G and db[N] (+)= sum_k G[k,:], with X
 * [K,M] (ldx) the layer input, G [K,N] (ldg) the output gradient, K the tokens.  db
 * NULL: weight only.  acc_w / acc_b: add to the gradient instead of overwriting it.
 * dtype_ab in {fp32, fp16, bf16, fp64}; dtype_w and dtype_b are fp32 or dtype_ab (fp64
 * for fp64).  fp16/bf16 GEMMs add up the column sums of G inside the GEMM; small
 * outputs split K, and one finishing launch reduces the weight and bias partials in
 * a fixed order (deterministic).  workspace: tg_gemm_wgrad_workspace(dtype_ab, M, N,
 * K, db != NULL) bytes, 16-byte aligned. */
size_t tg_gemm_wgrad_workspace(int dtype_ab, int64_t M, int64_t N, int64_t K, int with_bias);
int tg_gemm_wgrad(int dtype_ab, int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx,
                  const void* G, int64_t ldg, int dtype_w, void* dW, int64_t ldw, int acc_w,
                  int dtype_b, void* db, int acc_b, void* workspace, size_t workspace_bytes,
                  void* stream);
/* n weight (+ bias) gradients of the same shape, tg_gemm_wgrad for each member g:
 * dW[g] (+)= X[g]^T @ G[g], db[g] (+)= column sums of G[g] (db NULL or db[g] NULL: no
 * bias; acc_w / acc_b NULL: overwrite all).  X, G, dW, db, acc_w and acc_b are host
 * arrays of n entries.  The reference runs these products one node at a time in its
 * backward sweep (the matmul node of _core.py:1064-1068 for each Linear, _nn.py:258-285);
 * gathered, the equal-shaped layers' products (e.g. the q/k/v/o projections of every
 * block) become one launch of whole-K tiles, without the K split and finishing pass
 * that a lone small-output product needs.  fp16/bf16 groups whose tiles fill the CUs
 * take the grouped kernel; other members run through tg_gemm_wgrad one after another.
 * Every member's gradient buffers must be distinct.  workspace:
 * tg_gemm_wgrad_group_workspace(dtype_ab, n, M, N, K, any db[g] != NULL) bytes. */
size_t tg_gemm_wgrad_group_workspace(int dtype_ab, int n, int64_t M, int64_t N, int64_t K,
                                     int with_bias);
int tg_gemm_wgrad_group(int dtype_ab, int n, int64_t M, int64_t N, int64_t K,
                        const void* const* X, int64_t ldx, const void* const* G, int64_t ldg,
                        int dtype_w, void* const* dW, int64_t ldw, const int* acc_w,
                        int dtype_b, void* const* db, const int* acc_b, void* workspace,
                        size_t workspace_bytes, void* stream);
/* tg_gemm_wgrad_group over members of one input shape X[g]: (K, M) whose outputs
 * differ in width: G[g] is (K, N[g]) with row stride ldg[g], dW[g] (M, N[g]) with row
 * stride ldw[g] (N, ldg, ldw: host arrays of n entries).  The members' output tiles
 * form one launch, so layers of one input width (e.g. a fused Q/K/V projection, N =
 * 3d, and the output projection, N = d) fill the CUs together.  workspace:
 * tg_gemm_wgrad_group_n_workspace bytes. */
size_t tg_gemm_wgrad_group_n_workspace(int dtype_ab, int n, int64_t M, const int64_t* N,
                                       int64_t K, int with_bias);
int tg_gemm_wgrad_group_n(int dtype_ab, int n, int64_t M, const int64_t* N, int64_t K,
                          const void* const* X, int64_t ldx, const void* const* G,
                          const int64_t* ldg, int dtype_w, void* const* dW, const int64_t* ldw,
                          const int* acc_w, int dtype_b, void* const* db, const int* acc_b,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- attention ------------------------------------------------------------ */
/* FlashAttention forward on contiguous (B,H,S,D) tensors, saving the row
 * log-sum-exp lse[B,H,Sq] (fp32) for the backward.  causal masks col > row
 * (_core.py:1686-1786).  dtype fp32, fp16 or bf16; head dim D from 1 to 256 (fp16/bf16
 * with D 64 or 128 and 16-byte aligned operands run the tuned kernels, everything else
 * the generic ones on fp32 matrix cores); any B*H (split over launches of at most
 * 65535 heads), H <= 65535. */
int tg_flash_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                      int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D, float scale,
                      int causal, void* stream);
/* FlashAttention backward (_core.py:1799-1867): recomputes P from lse,
 * dV = P^T dO, dP = dO V^T, dS = P*(dP - rowsum(dO*O))*scale, dQ = dS K,
 * dK = dS^T Q.  Workspace from tg_flash_attn_bwd_workspace. */
size_t tg_flash_attn_bwd_workspace(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D);
int tg_flash_attn_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
                      const void* dout, const float* lse, void* dq, void* dk, void* dv, int64_t B,
                      int64_t H, int64_t Sq, int64_t Sk, int64_t D, float scale, int causal,
                      int accumulate, void* workspace, size_t workspace_bytes, void* stream);
/* Layout variants of the two calls above.  layout 0: q/k/v/o/dout/dq/dk/dv are
 * contiguous (B,H,S,D); layout 1: they are contiguous (B,S,H,D) in memory (the head
 * split of a (B,S,H*D) projection: the reference's reshape + transpose views before
 * flash_attention, _core.py:1686-1700), read and written in place of a transposing
 * copy.  lse and the workspace stay (B,H,S). */
int tg_flash_attn_fwd_layout(int dtype, const void* q, const void* k, const void* v, void* o,
                             float* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                             float scale, int causal, int layout, void* stream);
int tg_flash_attn_bwd_layout(int dtype, const void* q, const void* k, const void* v,
                             const void* o, const void* dout, const float* lse, void* dq,
                             void* dk, void* dv, int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                             int64_t D, float scale, int causal, int accumulate, int layout,
                             void* workspace, size_t workspace_bytes, void* stream);
/* Self-attention on one packed projection qkv of (B,S,3,H,D) memory: the output of a
 * fused Q/K/V Linear(d, 3*H*D) whose columns hold the query, key and value heads in that
 * order (the reference's MultiHeadAttention module projects x by w_q, w_k, w_v and splits
 * the heads by reshape + transpose copies, _training.py:1885-1904; _core.py:1873-1913 is
 * the functional form).  q, k and v are read in place (rows 3*H*D elements apart); o and
 * dout are (B,S,H,D) (the merged-head input of the output projection, with no copy); the
 * backward writes (or adds, accumulate != 0) dq, dk and dv into the matching columns of
 * dqkv, also (B,S,3,H,D).  lse (B,H,S) fp32; workspace as tg_flash_attn_bwd_workspace(B,
 * H, S, S, D).  Same dtypes and head dims as the calls above. */
int tg_flash_attn_fwd_qkv(int dtype, const void* qkv, void* o, float* lse, int64_t B, int64_t H,
                          int64_t S, int64_t D, float scale, int causal, void* stream);
int tg_flash_attn_bwd_qkv(int dtype, const void* qkv, const void* o, const void* dout,
                          const float* lse, void* dqkv, int64_t B, int64_t H, int64_t S,
                          int64_t D, float scale, int causal, int accumulate, void* workspace,
                          size_t workspace_bytes, void* stream);
/* FlashAttention on float64 data (the reference runs flash_attention in the input's
 * dtype, _core.py:1716-1867): the scores of a chunk of heads are materialised in the
 * workspace (as the reference materialises them per query block), the products run on
 * the fp64 matrix cores, softmax and lse (natural log, double, [B,H,Sq]) in double;
 * the backward recomputes P from lse and uses the reference's row term
 * dS = P*(dP - rowsum(P*dP))*scale.  layout as for the _layout forms; o is not read by
 * the backward.  Workspace: tg_flash_attn_f64_workspace bytes: 2*hc*Sq*Sk doubles for a chunk of hc
 * heads sized to about 512 MiB, but never less than one head's 2*Sq*Sk doubles (e.g.
 * 4 GiB at Sq = Sk = 16384). */
size_t tg_flash_attn_f64_workspace(int64_t B, int64_t H, int64_t Sq, int64_t Sk);
int tg_flash_attn_fwd_f64(const double* q, const double* k, const double* v, double* o,
                          double* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                          double scale, int causal, int layout, void* workspace,
                          size_t workspace_bytes, void* stream);
int tg_flash_attn_bwd_f64(const double* q, const double* k, const double* v, const double* o,
                          const double* dout, const double* lse, double* dq, double* dk,
                          double* dv, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                          double scale, int causal, int layout, int accumulate,
                          void* workspace, size_t workspace_bytes, void* stream);

/* A Linear layer's GEMM with a fused epilogue (fp16 / bf16 on the DMA-staged kernel;
 * other shapes, layouts or alignments return -3 and the caller runs the separate
 * kernels).  The product is rounded to the dtype exactly as tg_gemm stores it, then
 *   epi 1, GELU backward: C (+)= round(A B^T) * gelu'(X), A [M,K], B [N,K], X [M,N] the
 *     GELU input (ldx).  The input gradient of a Linear layer fed by a GELU with the
 *     GELU's backward applied (matmul bwd _core.py:1060 followed by the gelu closure
 *     _core.py:1185-1206); beta 0 overwrites C, 1 adds.
 *   epi 2, GELU forward: C = round(A B + bias), X = round(gelu(C)), B [K,N]: a Linear
 *     layer's forward (_nn.py:258-285) followed by gelu (_core.py:1172-1197), both
 *     outputs written.
 *   epi 3, residual: C = round(A B + bias) + X, B [K,N]: x + Linear(..) (__add__,
 *     _core.py:941-951, after _nn.py:258-285).
 * bias is fp32 [N] or null (null for epi 1).  Each result equals the separate kernels'
 * (tg_gemm / tg_gemm_bias, then tg_gelu_bwd / tg_gelu_fwd / the add) bit for bit. */
int tg_gemm_epilogue(int dtype, int epi, int64_t M, int64_t N, int64_t K, const void* A,
                     int64_t lda, const void* B, int64_t ldb, const float* bias, void* X,
                     int64_t ldx, float beta, void* C, int64_t ldc, void* stream);

/* Cross-entropy over logits [N, C] with int64 targets (CrossEntropyLoss,
 * _nn.py:1128-1185).  Forward: per-row log-sum-exp lse[N] and per-row loss
 * -log(p[t] + 1e-10) (label smoothing s: -sum_c w_c log(p_c + 1e-10), w = s/C +
 * (1-s) onehot); the caller reduces loss[N].  A target in [-C, 0) counts from the end
 * (the reference indexes with NumPy); one outside [-C, C) gives a NaN loss.  This holds
 * for every cross-entropy entry point.  dtype fp32/fp16/bf16 (fp64:
 * tg_cross_entropy_fwd_f64). */
int tg_cross_entropy_fwd(int dtype, const void* logits, const int64_t* targets, int64_t N,
                         int64_t C, float label_smoothing, float* lse, float* loss, void* stream);
/* tg_cross_entropy_fwd (label smoothing 0) and the gradient grad = (softmax - onehot) *
 * scale in the logits' dtype, from one read of the logits (each row held in registers;
 * C at most tg_cross_entropy_fwd_grad_max_classes(dtype), a multiple of 16 bytes' worth
 * of elements, 16-byte aligned logits and grad).  Bit for bit tg_cross_entropy_fwd
 * followed by tg_cross_entropy_bwd(accumulate = 0).  The reference's backward does not
 * use the loss's upstream gradient (_nn.py:1168-1180), so the gradient is known at the
 * forward (_nn.py:1128-1185) and the backward only hands it to the logits. */
int tg_cross_entropy_fwd_grad_max_classes(int dtype);
int tg_cross_entropy_fwd_grad(int dtype, const void* logits, const int64_t* targets, int64_t N,
                              int64_t C, float* lse, float* loss, float scale, void* grad,
                              void* stream);
/* Backward (_nn.py:1168-1180): grad (+)= (softmax(logits) - w) * scale, with
 * scale = 1/N for the mean reduction and no upstream-gradient factor, as in the
 * reference.  grad has dtype dtype_grad. */
int tg_cross_entropy_bwd(int dtype, const void* logits, const int64_t* targets, const float* lse,
                         int64_t N, int64_t C, float label_smoothing, float scale, int dtype_grad,
                         void* grad, int accumulate, void* stream);
/* The cross-entropy pair for fp64 logits, in double, with double scalars (label
 * smoothing and the gradient scale, e.g. 1/N, are not exact in fp32); lse and loss are
 * double and the gradient is fp64 (the reference's arithmetic on float64 logits). */
int tg_cross_entropy_fwd_f64(const double* logits, const int64_t* targets, int64_t N, int64_t C,
                             double label_smoothing, double* lse, double* loss, void* stream);
int tg_cross_entropy_bwd_f64(const double* logits, const int64_t* targets, const double* lse,
                             int64_t N, int64_t C, double label_smoothing, double scale,
                             double* grad, int accumulate, void* stream);

/* Embedding forward (Embedding.__call__, _nn.py:1076-1082): out[i, :] =
 * weight[indices[i], :] converted to dtype_out (the autocast cast of the gathered
 * rows folded into the gather).  Negative indices wrap by num_embeddings, as NumPy's;
 * rows of indices outside [-num_embeddings, num_embeddings) are written as zeros (the
 * caller checks host indices and raises IndexError, as the reference does). */
int tg_embedding_fwd(int dtype_w, const void* weight, const int64_t* indices, int64_t n_tokens,
                     int64_t dim, int64_t num_embeddings, int dtype_out, void* out,
                     void* stream);
/* Embedding backward (Embedding._backward, _nn.py:1083-1089): grad[idx[i]] (+)=
 * dout[i] for n_tokens rows of dim elements, grad [num_embeddings, dim].
 * Deterministic: each index's rows are summed in their original order (np.add.at's
 * order); up to 8192 tokens in one launch that writes every gradient row once, more
 * through a stable sort of the indices.  Indices in [-num_embeddings, 0) count from
 * the end (the reference's NumPy indexing); indices outside [-num_embeddings,
 * num_embeddings) are skipped.  Workspace from tg_embedding_bwd_workspace (0 bytes up to 8192 tokens). */
size_t tg_embedding_bwd_workspace(int64_t n_tokens, int64_t num_embeddings);
int tg_embedding_bwd(int dtype_dout, const void* dout, const int64_t* indices, int64_t n_tokens,
                     int64_t dim, int dtype_grad, void* grad, int64_t num_embeddings,
                     int accumulate, void* workspace, size_t workspace_bytes, void* stream);
/* dst[c][r] += alpha * src[r][c] for src [rows, cols] (sync_tied_gradients,
 * _training.py:264-284: source.grad += param.grad.T).  fp32/fp16/bf16 in fp32; when
 * either side is fp64 (fp64/fp64, fp64 into fp32, fp32 into fp64) in double, rounded
 * once to the destination. */
int tg_transpose_add(int dtype_src, const void* src, int64_t rows, int64_t cols, int dtype_dst,
                     void* dst, float alpha, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TGBWD_H */
