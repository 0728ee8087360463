#ifndef KVL_MLA_STATE_H
#define KVL_MLA_STATE_H

/* Expanded-K/V MLA state (correctness reference state of the runtime).
 * Struct layout byte-identical to include/kvl/mla_state.h:13-22 of the reference. */

#include <stddef.h>
#include "kvl/ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int capacity;
    int len;
    int num_heads;
    int qk_nope_dim;
    int qk_rope_dim;
    int v_head_dim;
    float *keys;   /* [capacity, num_heads, qk_nope_dim + qk_rope_dim] host */
    float *values; /* [capacity, num_heads, v_head_dim] host */
} KvlMlaState;

/* include/kvl/mla_state.h:24-27 */
int kvl_mla_state_init(KvlMlaState *state, const KvlMlaConfig *cfg, int capacity);
void kvl_mla_state_reset(KvlMlaState *state);
void kvl_mla_state_free(KvlMlaState *state);
size_t kvl_mla_state_bytes(const KvlMlaState *state);

/* include/kvl/mla_state.h:29-37 (src/mla_state.c:66-149). Non-absorbed decode of one
 * token at `position` (== state->len); appends its expanded K/V, then attends. */
int kvl_mla_decode_bf16(float *out, const float *x, int position,
                        const KvlMlaConfig *cfg, const KvlMlaBF16 *w, KvlMlaState *state);

#ifdef __cplusplus
}
#endif

#endif
