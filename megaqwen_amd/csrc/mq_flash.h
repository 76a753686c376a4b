// Unmasked [B, H, T, 64] attention (flash_attn.hip): host launcher.
#pragma once

#include <hip/hip_runtime.h>

// Workspace bytes for the K and V^T operand copies of [bh, T, 64] inputs.
size_t mq_flash_attn_workspace(int bh, int T);
// q, k, v, out: contiguous [bh, T, 64] 16-bit tensors (bf16, or fp16 if `f16`); bh <= 65535,
// T >= 1; workspace: mq_flash_attn_workspace(bh, T) bytes, 16-byte aligned.
// scale_log2 = softmax scale * log2(e).  Returns 0, or -1 if the launch failed.
int mq_launch_flash_attn_bhwd(const void* q, const void* k, const void* v, void* out, int bh,
                              int T, bool f16, float scale_log2, void* workspace,
                              hipStream_t stream);
