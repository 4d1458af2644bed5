"""tensor_gpu_v2 — MI355X backward-pass engine with the reference's API.

Drop-in for the gradient path of DragonShadows1978/Project-Tensor's tensor_gpu_v2:
`Tensor` and `Tensor.backward()`, `Linear`, `LayerNorm`, `BatchNorm2D`,
`FusedBatchNormReLU`, `flash_attention` (and `flash_attention_qkv` on a packed
projection), `Adam`/`AdamW`/`FusedAdam`,
`clip_grad_norm_`, `GradScaler` and `autocast`.  Gradient kernels are
hand-written HIP for gfx950 in libtgbwd.so, called over a ctypes C-ABI.
"""
from ._config import (autocast, enable_grad, enable_mixed_precision, get_default_dtype,
                      get_device, is_grad_enabled, is_mixed_precision, no_grad,
                      set_default_dtype, set_device, set_grad_enabled)
from ._core import (Tensor, flash_attention, flash_attention_qkv, memory_info,
                    multi_head_attention, scaled_dot_product_attention, sync)
from ._nn import (SGD, Adam, AdamW, BatchNorm2D, CrossEntropyLoss, Dropout, Embedding,
                  FusedBatchNormReLU, GradScaler, LayerNorm, Linear, Module, MSELoss,
                  clip_grad_norm_, clip_grad_value_)
from ._training import (CHECKPOINT_VERSION, FusedAdam, TiedWeight, load_checkpoint,
                        save_checkpoint, sync_tied_gradients, weight_tie)

__version__ = "2.0.0+mi355x"
