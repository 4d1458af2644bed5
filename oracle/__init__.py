"""CPU oracle for the tensor_gpu_v2 backward path — TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference's `device='cpu'` algorithms for
every function on the backward hot path (tensor_gpu_v2/_core.py, _nn.py,
_training.py of DragonShadows1978/Project-Tensor; each function cites the
reference lines it follows).  It is the parity checker for the HIP kernels and
the CPU baseline that bench.py times.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it; the product package never does.

Precision: every function computes in the dtype of its inputs (pass float64
arrays for a ground-truth reference, float32 to mimic the reference's fp32 CPU
arithmetic).

How each function is pinned (tests/test_oracle.py):
  gelu_bwd, silu_bwd            closed-form derivative vs central finite
                                differences (float64) and torch autograd float64
  softmax_fwd/bwd               torch.softmax autograd float64
  layernorm_fwd/bwd             torch.nn.functional.layer_norm autograd float64
  batchnorm_relu_fwd/bwd        torch batch_norm(training) + relu autograd float64
                                (the reference's BatchNorm2D oracle pattern)
  batchnorm_eval_fwd            eval mode with the running statistics set to the
                                batch's own equals the torch-pinned training path
  flash_attention_fwd/bwd       naive float64 softmax(QK^T s + mask) V autograd,
                                causal and non-causal, 3-D and 4-D inputs
  matmul_bwd / unbroadcast      torch autograd float64 over the reference test's
                                eight broadcast shape pairs, plus its error cases
                                and known answer (2,3,4)->(1,3,1) == 8
  adam_step                     hand-derived closed form at t = 1 and t = 2
  GradScalerRef, clip_grad_norm the reference tests' known answers (norm 13,
                                inf-norm 5, overflow 65536 -> 32768, growth after
                                the interval, min-scale clamp, NaN zeroing)
  cross_entropy_fwd/bwd         torch.nn.functional.cross_entropy autograd
                                float64 (mean reduction), upstream grad ignored
  embedding_bwd                 np.add.at closed form with repeated indices
  relu/leaky_relu/swish/sigmoid/tanh/exp/log/pow_bwd
                                torch autograd float64 of the same op, central
                                finite differences, and the kinks (relu at 0 -> 0,
                                leaky at 0 -> 1) by closed form
  log_softmax_fwd/bwd           torch.log_softmax autograd float64, any axis
  max_bwd                       torch.amax autograd float64 (ties share the
                                gradient evenly), axis None / int / keepdims
  getitem_bwd                   torch index backward (index_put accumulate),
                                integer arrays with repeats and boolean masks
No function is left unpinned.
"""
from .ref_ops import *  # noqa: F401,F403
