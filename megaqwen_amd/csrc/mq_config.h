// Compile-time layer shape of the kernels: the Qwen3-0.6B layer (csrc/megakernel/
// megakernel_kernels.py:13-21 of the reference).  Layer count, vocabulary size, maximum sequence
// length and prefill length are run-time values.
#pragma once

#define MQ_H 1024                       // hidden size
#define MQ_I 3072                       // SwiGLU intermediate size
#define MQ_NQ 16                        // query heads
#define MQ_NKV 8                        // key/value heads
#define MQ_D 128                        // head dim
#define MQ_GQA (MQ_NQ / MQ_NKV)         // query heads per kv head (2)
#define MQ_QDIM (MQ_NQ * MQ_D)          // 2048
#define MQ_KVDIM (MQ_NKV * MQ_D)        // 1024
#define MQ_QKV (MQ_QDIM + 2 * MQ_KVDIM) // 4096 rows of the fused q|k|v projection
#define MQ_EPS 1e-6f

#define MQ_THREADS 512                  // threads per workgroup of the decode kernels (8 waves)
#define MQ_WAVES (MQ_THREADS / 64)
#define MQ_CWAVES 7                     // compute waves; wave 7 is the sync wave (barrier + inputs)
#define MQ_SYNC_WAVE 7

#define MQ_MAX_CHUNKS 64                // attention split-K chunks per kv head (upper bound)
#define MQ_GROUP_CHUNKS 32              // split-K chunks of one kv-head group (decode kernel)
#define MQ_MAX_LAYERS 64                // decoder layers (the persistent kernel keeps their
                                        // weight-pointer table in LDS)
#define MQ_STEPS_PER_LAUNCH 64          // decode_steps: tokens chained inside one persistent launch
#define MQ_PART_STRIDE 132              // floats per attention partial: m, l, pad, pad, o[128]
#define MQ_ATT_BLOCK (32 * MQ_CWAVES)   // 224 positions scored per pass of a chunk (32 per wave)
#define MQ_ATT_SLOT (4 * MQ_CWAVES)     // 28: the smallest split-K chunk (4 positions per wave)
#define MQ_ATT_LOCAL_DEFAULT MQ_ATT_BLOCK   // default attn_local_max (persistent decode): local
                                             // attention while one 224-position block holds
                                             // the cache
#define MQ_GROUPS MQ_NKV                // persistent decode: workgroup wg serves kv head wg % 8
