// Unmasked [B, H, T, 64] attention (flash_attn.hip): host launcher.
#pragma once

#include <hip/hip_runtime.h>

// q, k, v, out: contiguous [bh, T, 64] 16-bit tensors (bf16, or fp16 if `f16`); bh <= 65535,
// T >= 1.  scale_log2 = softmax scale * log2(e).  Returns 0, or -1 if the launch failed.
int mq_launch_flash_attn_bhwd(const void* q, const void* k, const void* v, void* out, int bh,
                              int T, bool f16, float scale_log2, hipStream_t stream);
