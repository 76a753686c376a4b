// Prefill path: buffers carved from the decoder workspace and the host launcher (prefill.hip).
#pragma once

#include "mq_decode.h"

struct MqPrefillBuffers {
  int max_n;
  bf16_t* h;     // [n, H]    residual stream (bf16, as the reference's hidden_bf16)
  bf16_t* xn;    // [n, H]    RMSNorm output
  bf16_t* qkv;   // [n, 4096] q | k | v projections (q/k rotated in place)
  bf16_t* att;   // [n, 2048] attention output
  bf16_t* m;     // [n, 3072] silu(gate) * up
  bf16_t* vt;    // V^T of each kv head in attention-operand tile order (prefill.hip vt_index)
  bf16_t* kt;    // K of each kv head in attention-operand tile order (prefill.hip kt_index)
  int ntiles;    // 32-key tiles per kv head in vt / kt (max_n rounded up)
  float* part;   // split-K fp32 partials of the GEMMs (prefill.hip gemm_plan)
  uint32_t* cnt; // split-K arrival counters, one per output tile; zero between GEMMs (cleared
                 // with the decoder state, reset by the last split of each tile)
  size_t cnt_bytes;
};

size_t mq_prefill_workspace_bytes(int max_n);
void mq_prefill_bind(MqPrefillBuffers* b, char* base, int max_n);
// `host_layers` is the host copy of the device layer table p.layers.
// `patch` (optional, bf16 [patch_len, H]) replaces the embedding rows
// [patch_start, patch_start + patch_len), which must lie inside [0, n).
// `trace` (optional, bf16 [num_layers][n][H]) receives the residual stream after every layer.
int mq_launch_prefill(const MqDecodeParams& p, const MqLayerW* host_layers,
                      const MqPrefillBuffers& b, const int32_t* tokens, int n, int32_t* tok_out,
                      float* logits, int grid, hipStream_t stream, const bf16_t* patch = nullptr,
                      int patch_start = 0, int patch_len = 0, bf16_t* trace = nullptr);
