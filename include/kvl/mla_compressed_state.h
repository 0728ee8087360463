#ifndef KVL_MLA_COMPRESSED_STATE_H
#define KVL_MLA_COMPRESSED_STATE_H

/* Compressed FP32 latent history. Struct layout byte-identical to
 * include/kvl/mla_compressed_state.h:7-14 of the reference. The host arrays stay
 * authoritative: every call that appends rows also writes them back to these arrays. */

#include <stddef.h>
#include "kvl/ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int capacity;
    int len;
    int kv_lora_rank;
    int qk_rope_dim;
    float *latent; /* [capacity, kv_lora_rank] host */
    float *rope;   /* [capacity, qk_rope_dim] host, RoPE already applied */
} KvlMlaCompressedState;

/* include/kvl/mla_compressed_state.h:16-25 (src/mla_compressed_state.c:24-50) */
int kvl_mla_compressed_state_init(KvlMlaCompressedState *state, const KvlMlaConfig *cfg,
                                  int capacity);
void kvl_mla_compressed_state_reset(KvlMlaCompressedState *state);
int kvl_mla_compressed_state_truncate(KvlMlaCompressedState *state, int new_len);
void kvl_mla_compressed_state_free(KvlMlaCompressedState *state);
size_t kvl_mla_compressed_state_bytes(const KvlMlaCompressedState *state);

/* include/kvl/mla_compressed_state.h:27-31 (src/mla_compressed_state.c:52-84) */
int kvl_mla_compressed_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                          const KvlMlaBF16 *w, KvlMlaCompressedState *state);

/* include/kvl/mla_compressed_state.h:33-38 (src/mla_compressed_state.c:86-161) */
int kvl_mla_decode_compressed_bf16(float *out, const float *x, int position,
                                   const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                   KvlMlaCompressedState *state);

/* include/kvl/mla_compressed_state.h:40-46 (src/mla_compressed_state.c:163-184).
 * Decode of `count` tokens of one sequence, equal bit for bit to `count` single-token decodes
 * (the reference loops them): the tokens run as one batch whose members share the state, each
 * computed as a lone decode at its position would be. */
int kvl_mla_decode_compressed_block_bf16(float *out, const float *x, int count,
                                         int start_position, const KvlMlaConfig *cfg,
                                         const KvlMlaBF16 *w, KvlMlaCompressedState *state);

#ifdef __cplusplus
}
#endif

#endif
