/* CPU oracle of the MLA hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference runtime's MLA arithmetic, used by tests/ as the
 * parity checker and by bench.py as the CPU baseline when the reference build under
 * oracle/_ref is absent. Nothing in the product library links or calls this code.
 *
 * Every function names the reference file:line it restates. Summation orders follow the
 * reference exactly (double accumulation where the reference uses double; the AVX2 8-lane
 * FP32 GEMV order and the AVX2 2x4-lane double dot order are emulated lane by lane), so the
 * oracle reproduces the reference bit for bit when both are built without FP contraction.
 *
 * Functions use the same public state structs as the library headers under include/kvl. */
#ifndef KVL_ORACLE_H
#define KVL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "kvl/ops.h"
#include "kvl/mla_state.h"
#include "kvl/mla_compressed_state.h"
#include "kvl/mla_compressed_q8_state.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Summation order of the GEMV and of the streaming-prefill dot products.
 *   ORC_ORDER_SCALAR: the reference built without KVL_USE_AVX2 (src/ops.c:19-24,
 *                     src/mla_prefill_streaming.c:54-58).
 *   ORC_ORDER_AVX2:   the reference built with KVL_USE_AVX2 (src/ops.c:31-50,
 *                     src/mla_prefill_streaming.c:32-53). */
enum { ORC_ORDER_SCALAR = 0, ORC_ORDER_AVX2 = 1 };
void orc_set_order(int order);
int orc_get_order(void);

/* Bit helpers: src/ops.c:12-17, src/mla_compressed_q8_state.c:9-16. */
float orc_bf16_to_f32(uint16_t x);
uint16_t orc_f32_to_bf16_rne(float x);

/* src/ops.c:53-66 (OpenMP over rows when out > 64, as the reference). */
void orc_matvec_bf16(float *y, const float *x, const uint16_t *w, int in, int out);
/* src/ops.c:76-83 */
void orc_rmsnorm_bf16(float *y, const float *x, const uint16_t *weight, int n, float eps);
/* src/mla_compressed_q8_state.c:18-32 (same formula at src/ops.c:89-103, src/mla_state.c:8-22,
 * src/mla_compressed_state.c:8-22, src/mla_prefill_streaming.c:15-29). */
void orc_rope_interleaved(float *dst, const float *raw, int dim, int position, float theta);
/* src/mla_compressed_q8_state.c:34-55 */
void orc_quantize_latent(int8_t *dst, float *scale_out, const float *src, int n);
/* src/mla_compressed_q8_state.c:57-61 */
float orc_dequant(int8_t q, float scale);
/* One Q8 history row from the kv_a output of a token (src/mla_compressed_q8_state.c:111-127,
 * after the GEMV): RMSNorm -> quantize, RoPE -> BF16 RNE. katmp is [R + DR]. */
void orc_q8_row_from_katmp(int8_t *codes, float *scale, uint16_t *rope_bf16, const float *katmp,
                           const uint16_t *kv_a_norm, int R, int DR, float eps, int position,
                           float theta);
/* The quantizer-boundary form used for bit-exact checks: latent [R] (already normalised) and
 * raw k_rope [DR] (before RoPE) -> codes, scale, BF16 RoPE row. */
void orc_q8_pack_row(int8_t *codes, float *scale, uint16_t *rope_bf16, const float *latent,
                     const float *k_rope_raw, int R, int DR, int position, float theta);

/* Expanded state: src/mla_state.c:24-149 */
int orc_mla_state_init(KvlMlaState *s, const KvlMlaConfig *cfg, int capacity);
void orc_mla_state_reset(KvlMlaState *s);
void orc_mla_state_free(KvlMlaState *s);
size_t orc_mla_state_bytes(const KvlMlaState *s);
int orc_mla_decode_bf16(float *out, const float *x, int position, const KvlMlaConfig *cfg,
                        const KvlMlaBF16 *w, KvlMlaState *s);

/* Compressed FP32 state: src/mla_compressed_state.c:24-184 */
int orc_mla_compressed_state_init(KvlMlaCompressedState *s, const KvlMlaConfig *cfg, int capacity);
void orc_mla_compressed_state_reset(KvlMlaCompressedState *s);
int orc_mla_compressed_state_truncate(KvlMlaCompressedState *s, int new_len);
void orc_mla_compressed_state_free(KvlMlaCompressedState *s);
size_t orc_mla_compressed_state_bytes(const KvlMlaCompressedState *s);
int orc_mla_compressed_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                          const KvlMlaBF16 *w, KvlMlaCompressedState *s);
int orc_mla_decode_compressed_bf16(float *out, const float *x, int position,
                                   const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                   KvlMlaCompressedState *s);
/* The FP32 decode with the appended row rounded to bf16 before it is stored and attended: the
 * library's BF16-latent history, restated over an FP32 state of bf16 values. */
int orc_mla_decode_compressed_bf16_rows(float *out, const float *x, int position,
                                        const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                        KvlMlaCompressedState *s);
int orc_mla_decode_compressed_block_bf16(float *out, const float *x, int count, int start_position,
                                         const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                         KvlMlaCompressedState *s);

/* Compressed Q8 state: src/mla_compressed_q8_state.c:63-255 */
int orc_mla_compressed_q8_state_init(KvlMlaCompressedQ8State *s, const KvlMlaConfig *cfg,
                                     int capacity);
void orc_mla_compressed_q8_state_reset(KvlMlaCompressedQ8State *s);
int orc_mla_compressed_q8_state_truncate(KvlMlaCompressedQ8State *s, int new_len);
void orc_mla_compressed_q8_state_free(KvlMlaCompressedQ8State *s);
size_t orc_mla_compressed_q8_state_bytes(const KvlMlaCompressedQ8State *s);
int orc_mla_compressed_q8_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                             const KvlMlaBF16 *w, KvlMlaCompressedQ8State *s);
int orc_mla_decode_compressed_q8_bf16(float *out, const float *x, int position,
                                      const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                      KvlMlaCompressedQ8State *s);

/* Causal prefill: head-streaming form (src/mla_prefill_streaming.c:78-206) and the
 * fully-materialised form kept by the reference as a lab oracle (src/ops.c:105-192). */
int orc_mla_prefill_streaming(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg,
                              const KvlMlaBF16 *w);
int orc_mla_prefill_materialized(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg,
                                 const KvlMlaBF16 *w);
/* Selected query rows of the streaming prefill (out [nrows, H], row i = query row rows[i]),
 * each bit-identical to that row of orc_mla_prefill_streaming: a checker for long prefills. */
int orc_mla_prefill_streaming_rows(float *out, const float *x, int seq_len, const int *rows,
                                   int nrows, const KvlMlaConfig *cfg, const KvlMlaBF16 *w);

#ifdef __cplusplus
}
#endif

#endif
