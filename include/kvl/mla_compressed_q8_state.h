#ifndef KVL_MLA_COMPRESSED_Q8_STATE_H
#define KVL_MLA_COMPRESSED_Q8_STATE_H

/* Row-wise Q8 latent history: per token 512 int8 codes, one FP32 scale and a BF16 RoPE
 * key (644 B at the Kimi-VL shapes). Struct layout byte-identical to
 * include/kvl/mla_compressed_q8_state.h:8-16 of the reference. */

#include <stddef.h>
#include <stdint.h>
#include "kvl/ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int capacity;
    int len;
    int kv_lora_rank;
    int qk_rope_dim;
    int8_t *latent_q8;     /* [capacity, kv_lora_rank] host */
    float *latent_scale;   /* [capacity] host */
    uint16_t *rope_bf16;   /* [capacity, qk_rope_dim] host, RoPE applied, BF16 RNE */
} KvlMlaCompressedQ8State;

/* include/kvl/mla_compressed_q8_state.h:18-25 (src/mla_compressed_q8_state.c:63-109) */
int kvl_mla_compressed_q8_state_init(KvlMlaCompressedQ8State *state, const KvlMlaConfig *cfg,
                                     int capacity);
void kvl_mla_compressed_q8_state_reset(KvlMlaCompressedQ8State *state);
int kvl_mla_compressed_q8_state_truncate(KvlMlaCompressedQ8State *state, int new_len);
void kvl_mla_compressed_q8_state_free(KvlMlaCompressedQ8State *state);
size_t kvl_mla_compressed_q8_state_bytes(const KvlMlaCompressedQ8State *state);

/* include/kvl/mla_compressed_q8_state.h:27-31 (src/mla_compressed_q8_state.c:129-159) */
int kvl_mla_compressed_q8_state_prefill_bf16(const float *x, int seq_len,
                                             const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                             KvlMlaCompressedQ8State *state);

/* include/kvl/mla_compressed_q8_state.h:33-38 (src/mla_compressed_q8_state.c:161-255) */
int kvl_mla_decode_compressed_q8_bf16(float *out, const float *x, int position,
                                      const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                      KvlMlaCompressedQ8State *state);

#ifdef __cplusplus
}
#endif

#endif
