// Prefill (placeholder until the MFMA path lands): reports "unsupported".
#include "mq_prefill.h"

static size_t pf_align(size_t v) { return (v + 255) / 256 * 256; }

size_t mq_prefill_workspace_bytes(int max_n) {
  if (max_n <= 0) return 0;
  const size_t n = (size_t)max_n;
  return pf_align(n * MQ_H * 2) * 2 + pf_align(n * MQ_QKV * 2) + pf_align(n * MQ_QDIM * 2) +
         pf_align(n * MQ_I * 2);
}

void mq_prefill_bind(MqPrefillBuffers* b, char* base, int max_n) {
  b->max_n = max_n;
  if (max_n <= 0) {
    b->h = b->xn = b->qkv = b->att = b->m = nullptr;
    return;
  }
  const size_t n = (size_t)max_n;
  char* c = base;
  b->h = reinterpret_cast<bf16_t*>(c);   c += pf_align(n * MQ_H * 2);
  b->xn = reinterpret_cast<bf16_t*>(c);  c += pf_align(n * MQ_H * 2);
  b->qkv = reinterpret_cast<bf16_t*>(c); c += pf_align(n * MQ_QKV * 2);
  b->att = reinterpret_cast<bf16_t*>(c); c += pf_align(n * MQ_QDIM * 2);
  b->m = reinterpret_cast<bf16_t*>(c);
}

int mq_launch_prefill(const MqDecodeParams&, const MqPrefillBuffers&, const int32_t*, int,
                      int32_t*, float*, int, hipStream_t) {
  return -1;
}
