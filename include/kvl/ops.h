#ifndef KVL_OPS_H
#define KVL_OPS_H

/* MLA subset of the runtime's numeric API, served by libkvl_mla (MI355X / gfx950).
 *
 * Struct layouts are byte-identical to the reference declarations so a caller built
 * against either header links against this library unchanged:
 *   KvlMlaConfig  <- include/kvl/ops.h:17-26
 *   KvlMlaBF16    <- include/kvl/ops.h:28-34
 * The MoE/router/MLP declarations of the reference header are not part of this library. */

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int hidden_size;
    int num_heads;
    int qk_nope_dim;
    int qk_rope_dim;
    int v_head_dim;
    int kv_lora_rank;
    float rms_eps;
    float rope_theta;
} KvlMlaConfig;

/* Row-major [out,in] BF16 matrices (kv_a_norm is a [kv_lora_rank] vector).
 * The pointers are borrowed for the duration of a call. */
typedef struct {
    const uint16_t *q_proj;    /* [num_heads*(qk_nope+qk_rope), hidden]            */
    const uint16_t *kv_a_proj; /* [kv_lora_rank+qk_rope, hidden]                   */
    const uint16_t *kv_a_norm; /* [kv_lora_rank]                                   */
    const uint16_t *kv_b_proj; /* [num_heads*(qk_nope+v_head), kv_lora_rank]       */
    const uint16_t *o_proj;    /* [hidden, num_heads*v_head]                        */
} KvlMlaBF16;

/* Replaces src/ops.c:12-17 (BF16 bits -> FP32). Pure host bit operation. */
float kvl_bf16_to_f32(uint16_t x);

/* Replaces src/ops.c:53-66. y[out] = W[out,in] . x[in]; host buffers, computed on the GPU
 * (FP32 accumulation). */
void kvl_matvec_bf16(float *y, const float *x, const uint16_t *w, int in, int out);

/* Replaces src/ops.c:76-83. y = x * (1/sqrtf(mean(x^2)+eps)) * w; host buffers, computed
 * on the GPU. */
void kvl_rmsnorm_bf16(float *y, const float *x, const uint16_t *weight, int n, float eps);

/* Replaces src/mla_prefill_streaming.c:78-206 (declared at include/kvl/ops.h:63-64).
 * Causal MLA prefill of seq_len tokens, x already input-RMS-normalised; out [seq_len, hidden].
 * Returns 0, or -1 on invalid arguments or a device error. */
int kvl_mla_prefill_bf16(float *out, const float *x, int seq_len,
                         const KvlMlaConfig *cfg, const KvlMlaBF16 *w);

#ifdef __cplusplus
}
#endif

#endif
