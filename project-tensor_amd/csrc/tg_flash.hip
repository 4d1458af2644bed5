// FlashAttention forward/backward (placeholder until the MFMA kernels land).
#include "tg_common.h"

TG_EXPORT int tg_flash_attn_fwd(int, const void*, const void*, const void*, void*, float*, int64_t,
                                int64_t, int64_t, int64_t, int64_t, float, int, void*) {
  tg_set_error("tg_flash_attn_fwd: not implemented");
  return TG_ERR_UNSUPPORTED;
}
TG_EXPORT size_t tg_flash_attn_bwd_workspace(int64_t, int64_t, int64_t, int64_t, int64_t) { return 0; }
TG_EXPORT int tg_flash_attn_bwd(int, const void*, const void*, const void*, const void*, const void*,
                                const float*, void*, void*, void*, int64_t, int64_t, int64_t, int64_t,
                                int64_t, float, int, int, void*, size_t, void*) {
  tg_set_error("tg_flash_attn_bwd: not implemented");
  return TG_ERR_UNSUPPORTED;
}
