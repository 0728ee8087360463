#ifndef KVL_MLA_HIP_H
#define KVL_MLA_HIP_H

/* Extensions of libkvl_mla (MI355X / gfx950) with no counterpart in the reference runtime.
 *
 * The reference MLA API (include/kvl/ops.h, mla_state.h, mla_compressed_state.h,
 * mla_compressed_q8_state.h) keeps its exact semantics: host buffers in and out, host
 * state arrays authoritative, synchronous calls. These extensions add what a GPU library
 * needs on top of it:
 *   - a BF16-latent history state (1152 B per row at the Kimi-VL shapes);
 *   - pinned device copies of a layer's weights (the reference borrows them per call);
 *   - explicit re-synchronisation of a state whose rows were edited in place on the host;
 *   - batched (ragged) decode over many sequences in one call;
 *   - stream-ordered device-pointer variants (no host sync), capturable in a HIP graph;
 *   - the quantiser boundary (fp32 latent -> Q8 row) as a standalone entry point;
 *   - device-side synthetic histories for benchmarks.
 * Every int-returning function returns 0 on success and -1 on failure; the reason is then
 * available from kvl_mla_last_error() (thread-local). Nothing here calls exit(). */

#include <stddef.h>
#include <stdint.h>

#include "kvl/mla_compressed_q8_state.h"
#include "kvl/mla_compressed_state.h"
#include "kvl/mla_state.h"
#include "kvl/ops.h"

#ifdef __cplusplus
extern "C" {
#endif

/* BF16-latent history: the layout of the FP32 compressed state (include/kvl/
 * mla_compressed_state.h:7-14 of the reference) with each normalised latent row and each rotated
 * RoPE key stored as bf16, rounded to nearest even with the rule of
 * src/mla_compressed_q8_state.c:9-16 (Inf/NaN words truncated): 2 * (kv_lora_rank + qk_rope_dim)
 * bytes per row, 1152 B at kv_lora_rank 512 / qk_rope_dim 64, half the FP32 state's 2304 B.
 * Decoding it computes the reference's FP32 decode (src/mla_compressed_state.c:86-161) over the
 * bf16-rounded rows. The host arrays stay authoritative as for the reference's states. */
typedef struct {
    int capacity;
    int len;
    int kv_lora_rank;
    int qk_rope_dim;
    uint16_t *latent; /* [capacity, kv_lora_rank] host, bf16 */
    uint16_t *rope;   /* [capacity, qk_rope_dim] host, bf16, RoPE already applied */
} KvlMlaCompressedBF16State;

/* Life cycle, with the checks and return values of the FP32 state's
 * (src/mla_compressed_state.c:24-50): init allocates zeroed host arrays (capacity > 0,
 * qk_rope_dim even); truncate needs 0 <= new_len <= len; bytes counts the struct and the arrays. */
int kvl_mla_compressed_bf16_state_init(KvlMlaCompressedBF16State *state, const KvlMlaConfig *cfg,
                                       int capacity);
void kvl_mla_compressed_bf16_state_reset(KvlMlaCompressedBF16State *state);
int kvl_mla_compressed_bf16_state_truncate(KvlMlaCompressedBF16State *state, int new_len);
void kvl_mla_compressed_bf16_state_free(KvlMlaCompressedBF16State *state);
size_t kvl_mla_compressed_bf16_state_bytes(const KvlMlaCompressedBF16State *state);
/* State prefill (src/mla_compressed_state.c:52-84 with bf16 rows): empty state, seq_len <=
 * capacity. */
int kvl_mla_compressed_bf16_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                               const KvlMlaBF16 *w, KvlMlaCompressedBF16State *state);
/* One decode token (src/mla_compressed_state.c:86-161 with the appended row stored as bf16):
 * position must equal len; host buffers, synchronous, host rows written. */
int kvl_mla_decode_compressed_bf16_bf16(float *out, const float *x, int position, const KvlMlaConfig *cfg,
                                        const KvlMlaBF16 *w, KvlMlaCompressedBF16State *state);
/* count tokens at start_position (= len) .. + count - 1, equal bit for bit to count single-token
 * decodes (src/mla_compressed_state.c:163-184 loops them). */
int kvl_mla_decode_compressed_bf16_block_bf16(float *out, const float *x, int count, int start_position,
                                              const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                              KvlMlaCompressedBF16State *state);

/* Last error of the calling thread ("" when none). */
const char *kvl_mla_last_error(void);

/* Optional explicit initialisation on the current HIP device (otherwise lazy). */
int kvl_mla_init(void);

/* Uploads the five weight arrays of a layer and pins the device copies under their host
 * addresses, so later calls with the same KvlMlaBF16 skip the content check; release them
 * before freeing or reusing the host arrays. Unpinned weights are cached by address, size
 * and a digest of 18 sampled 64-byte windows, and re-uploaded when that digest changes: an
 * in-place edit outside the sampled windows is not seen, so callers that edit weights in
 * place bind them or release them after the edit. */
int kvl_mla_bind_weights(const KvlMlaConfig *cfg, const KvlMlaBF16 *w);
int kvl_mla_release_weights(const KvlMlaBF16 *w);

/* Forces a full re-upload of rows [0, len) on the next call (for callers that overwrite
 * history rows below len in place, without truncate/reset). */
int kvl_mla_compressed_state_sync(KvlMlaCompressedState *state);
int kvl_mla_compressed_q8_state_sync(KvlMlaCompressedQ8State *state);
int kvl_mla_state_sync(KvlMlaState *state);
int kvl_mla_compressed_bf16_state_sync(KvlMlaCompressedBF16State *state);

/* One decode token for each of `batch` sequences: x [batch, hidden], out [batch, hidden],
 * positions[i] must equal states[i]->len (the reference rule, checked for every sequence
 * before anything runs). Host buffers; synchronous; host rows written back. */
int kvl_mla_decode_compressed_batch_bf16(float *out, const float *x, const int *positions,
                                         int batch, const KvlMlaConfig *cfg,
                                         const KvlMlaBF16 *w,
                                         KvlMlaCompressedState *const *states);
int kvl_mla_decode_compressed_q8_batch_bf16(float *out, const float *x, const int *positions,
                                            int batch, const KvlMlaConfig *cfg,
                                            const KvlMlaBF16 *w,
                                            KvlMlaCompressedQ8State *const *states);
int kvl_mla_decode_compressed_bf16_batch_bf16(float *out, const float *x, const int *positions,
                                              int batch, const KvlMlaConfig *cfg,
                                              const KvlMlaBF16 *w,
                                              KvlMlaCompressedBF16State *const *states);

/* Block decode over the Q8 history, the counterpart of kvl_mla_decode_compressed_block_bf16
 * (which the reference defines for the FP32 state only, src/mla_compressed_state.c:163-184):
 * count tokens at positions start_position .. start_position + count - 1 (start_position must
 * equal len). Outputs and appended rows equal those of count single-token decodes bit for bit;
 * the tokens share launches and history reads. */
int kvl_mla_decode_compressed_q8_block_bf16(float *out, const float *x, int count,
                                            int start_position, const KvlMlaConfig *cfg,
                                            const KvlMlaBF16 *w, KvlMlaCompressedQ8State *state);

/* Flags of the device-pointer variants. */
#define KVL_MLA_RESIDUAL 1u   /* out += attention(x) instead of out = attention(x)      */
#define KVL_MLA_NO_ADVANCE 2u /* append at position len but leave len (and host rows)  */

/* Stream-ordered variants: d_x / d_out are device pointers ([batch, hidden] fp32, d_out may
 * equal d_x with KVL_MLA_RESIDUAL), the call returns after enqueueing on kvl_mla_stream().
 * The appended rows stay on the device (host rows are not written); len advances unless
 * KVL_MLA_NO_ADVANCE. Weights must be bound. No allocation happens once the workspace has
 * grown to the batch size, so a warm call can be captured in a HIP graph. */
int kvl_mla_decode_compressed_q8_batch_device(float *d_out, const float *d_x, int batch,
                                              const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                              KvlMlaCompressedQ8State *const *states,
                                              unsigned flags);
int kvl_mla_decode_compressed_batch_device(float *d_out, const float *d_x, int batch,
                                           const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                           KvlMlaCompressedState *const *states,
                                           unsigned flags);
int kvl_mla_decode_compressed_bf16_batch_device(float *d_out, const float *d_x, int batch,
                                                const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                                KvlMlaCompressedBF16State *const *states,
                                                unsigned flags);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). The same computation and
 * results, bit for bit, as kvl_mla_decode_compressed_q8_batch_device, but every buffer beyond
 * the inputs, outputs, bound weights and state copies (the decode workspace and the split-K
 * partials) lives in one fixed device array of 24 MiB per GPU, and the call makes no
 * hipMalloc / hipFree. Limits, each rejected with -1 and a message: batch <= 16; the dims of
 * the MFMA route (16 heads, kv_lora_rank 512, qk_rope_dim 64); a split plan whose partials fit
 * the array (about 21 MiB, i.e. ~650 splits: e.g. 16 x 40K or 8 x 80K rows); weights bound;
 * each state's rows [0, len) already on the device (an allocating call or *_fill_synthetic
 * put them there); the RoPE table already covering the positions (an allocating decode at the
 * same or a later position built it). All calls on one GPU share the array: calls that overlap
 * in time on that GPU (a captured graph launched on another stream while a call runs) race. */
int kvl_mla_decode_compressed_q8_batch_device_noalloc(float *d_out, const float *d_x, int batch,
                                                      const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                                      KvlMlaCompressedQ8State *const *states,
                                                      unsigned flags);

/* The attention half of a decoder layer, as src/generate.c:34-67 (attention_token) computes it
 * for one token, for a batch over device buffers:
 *   n1 = RMSNorm(h, input_norm); h += attention(n1) (appending each sequence's row);
 *   n2 = RMSNorm(h, post_attn_norm).
 * d_h [batch, hidden] is the residual stream (in/out), d_n2 [batch, hidden] receives the MLP
 * input (must not alias d_h). The norms round as kvl_rmsnorm_bf16; the residual add is
 * h[i] + attn[i] in fp32 as the reference's. input_norm / post_attn_norm: bf16 [hidden] host
 * arrays (cached on the device like the weights). flags: 0 or KVL_MLA_NO_ADVANCE. Capturable
 * once warm, like the decode variants. */
int kvl_mla_attention_layer_q8_device(float *d_h, float *d_n2, int batch, const KvlMlaConfig *cfg,
                                      const KvlMlaBF16 *w, const uint16_t *input_norm,
                                      const uint16_t *post_attn_norm,
                                      KvlMlaCompressedQ8State *const *states, unsigned flags);
int kvl_mla_attention_layer_device(float *d_h, float *d_n2, int batch, const KvlMlaConfig *cfg,
                                   const KvlMlaBF16 *w, const uint16_t *input_norm,
                                   const uint16_t *post_attn_norm, KvlMlaCompressedState *const *states,
                                   unsigned flags);
int kvl_mla_attention_layer_bf16_device(float *d_h, float *d_n2, int batch, const KvlMlaConfig *cfg,
                                        const KvlMlaBF16 *w, const uint16_t *input_norm,
                                        const uint16_t *post_attn_norm,
                                        KvlMlaCompressedBF16State *const *states, unsigned flags);

/* Stream-ordered causal prefill over device buffers (d_x, d_out [seq_len, hidden] fp32);
 * same arithmetic as kvl_mla_prefill_bf16.
 * Range: the MFMA route (the Kimi-VL shapes) runs the attention on fp16/bf8 operands. Its
 * accuracy bound holds while every query row's largest attention logit (scale included) stays
 * within 512 in magnitude and the operands are finite in fp16. The host-buffer entry points
 * (kvl_mla_prefill_bf16 and the prefill-with-state-fill calls) check every call and compute
 * the output of a call outside that range again on the fp32 route, so they always return the
 * reference's result. A stream-ordered call outside that range writes NaN to d_out and raises
 * a flag that kvl_mla_prefill_range_status() reports. */
int kvl_mla_prefill_device(float *d_out, const float *d_x, int seq_len, const KvlMlaConfig *cfg,
                           const KvlMlaBF16 *w);

/* No counterpart in the reference (the C path computes in fp32/double throughout): whether any
 * stream-ordered prefill (kvl_mla_prefill_device, kvl_mla_prefill_compressed*_state_device)
 * since the previous call met query rows outside the MFMA route's range (its output is then
 * NaN). Synchronises the library stream; returns 0 (none), 1 (at least one; the flag is then
 * cleared and kvl_mla_last_error() says why) or -1. */
int kvl_mla_prefill_range_status(void);

/* Prefill with the state fill of the same tokens, as src/generate.c:208-210 sequences them
 * (kvl_mla_prefill_bf16(out, x, ...), then kvl_mla_compressed[_q8]_state_prefill_bf16(x, ...)),
 * with the same argument checks (state empty, seq_len <= capacity). The state (rows
 * [0, seq_len), len = seq_len) equals the state prefill's bit for bit. One upload of x; where
 * the shapes allow it (hidden 2048 or 4096 on the MFMA route) the prefill computes its kv_a
 * projection in the decode's summation order and both its attention and the state rows use
 * that one projection, so out equals kvl_mla_prefill_bf16's up to the rounding of kv_a
 * (kvl_mla_prefill_bf16 sums it inside its q GEMM); otherwise out is bit-identical and the
 * fill computes its own kv_a from the uploaded x. Synchronous; host rows written. */
int kvl_mla_prefill_compressed_state_bf16(float *out, const float *x, int seq_len,
                                          const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                          KvlMlaCompressedState *state);
int kvl_mla_prefill_compressed_q8_state_bf16(float *out, const float *x, int seq_len,
                                             const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                             KvlMlaCompressedQ8State *state);
/* The same over device buffers (d_x, d_out [seq_len, hidden] fp32), stream-ordered on
 * kvl_mla_stream(): the rows stay on the device (host rows are written only by *_pull); len is
 * set to seq_len. Not capturable (the fill may grow its workspace). */
int kvl_mla_prefill_compressed_state_device(float *d_out, const float *d_x, int seq_len,
                                            const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                            KvlMlaCompressedState *state);
int kvl_mla_prefill_compressed_q8_state_device(float *d_out, const float *d_x, int seq_len,
                                               const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                               KvlMlaCompressedQ8State *state);
/* The same pair for the BF16-latent state (rows bit-identical to its state prefill's). */
int kvl_mla_prefill_compressed_bf16_state_bf16(float *out, const float *x, int seq_len,
                                               const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                               KvlMlaCompressedBF16State *state);
int kvl_mla_prefill_compressed_bf16_state_device(float *d_out, const float *d_x, int seq_len,
                                                 const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                                 KvlMlaCompressedBF16State *state);

/* The library's HIP stream (hipStream_t) and helpers for callers without a HIP binding.
 * kvl_mla_synchronize waits for the stream; it returns -1 when a stream-ordered fused decode
 * enqueued since the last check had one of its bounded device waits time out (its outputs are
 * invalid; kvl_mla_last_error says so). */
void *kvl_mla_stream(void);
int kvl_mla_synchronize(void);
void *kvl_mla_device_alloc(size_t bytes);
int kvl_mla_device_free(void *p);
int kvl_mla_copy_to_device(void *dst, const void *src, size_t bytes);
int kvl_mla_copy_to_host(void *dst, const void *src, size_t bytes);
/* HIP graph capture of the calls made between begin and end on kvl_mla_stream(). A replay
 * repeats the captured calls exactly (positions, lengths, buffers). kvl_mla_graph_launch()
 * returns -1 when library-owned device memory was released or reallocated after the capture
 * (workspace or RoPE-table growth, a state freed or re-initialised, weights released), since
 * the graph may point into it; capture again then. */
int kvl_mla_capture_begin(void);
int kvl_mla_capture_end(void **graph_exec);
int kvl_mla_graph_launch(void *graph_exec);
int kvl_mla_graph_destroy(void *graph_exec);

/* Measurement helpers. kvl_mla_timing_enable(1) brackets every decode-step kernel with HIP
 * events on kvl_mla_stream() (not during graph capture); kvl_mla_timing_enable(2) also
 * records the events into a graph being captured (event-record nodes: each replay of that
 * graph overwrites their timestamps, so read once after the last replay, then destroy the
 * graph before timing anything else). kvl_mla_timing_read() sums the
 * durations (ms) and launch counts of the six stages (gemv_in, append [+ qprep: one launch
 * for the compressed formats], qprep [expanded format], attention,
 * combine, gemv_out) since the last read. kvl_mla_timing_stages(mask) limits the bracketing
 * to the stages whose bit is set (bit i: stage i; all six by default): every bracketed launch
 * carries its two event records, whose gaps the durations include. Events: record on the
 * library stream, elapsed time between two recorded events (waits for the second).
 * kvl_mla_copy_kernel: a plain 16-byte vector copy kernel (bytes % 16 == 0), for calibrating
 * memory counters. */
int kvl_mla_timing_enable(int on);
/* Form of the Q8 decode of two or more independent sequences at the Kimi shapes (library
 * extension, no counterpart in the reference): on = 1 (the default) prepares the queries and
 * appends the rows inside the attention launch, on = 0 in a launch of their own before it (the
 * form the block decode and the no-allocation entry point always use). The results are the same
 * bit for bit. Returns the previous setting, or -1. The environment variable
 * KVL_MLA_NO_FUSED_QPREP=1 sets 0 at initialisation. */
int kvl_mla_set_fused_qprep(int on);
/* Extension, no counterpart in the reference. Where the fused form above runs for eight
 * sequences with equal split counts (the batch-8 decode of long histories), the attention launch
 * also merges the split partials and applies W_UV (the combine), each sequence's splits placed on
 * one XCD so that its partials are read from that XCD's L2; 0 keeps the combine in a launch of
 * its own. The results are the same bit for bit. Returns the previous setting, or -1.
 * KVL_MLA_NO_FUSED_COMBINE=1 sets 0 at initialisation. */
int kvl_mla_set_fused_combine(int on);
/* Extension, no counterpart in the reference. Where the fused form runs for at most eight
 * sequences over at least 232 splits, the attention launch also computes the q_proj | kv_a
 * projection (its first 232 workgroups each take one block of the projection GEMV, and the query
 * preparation and the append wait for the blocks they read); 0 keeps the projection in a launch
 * of its own. The results are the same bit for bit. Returns the previous setting, or -1.
 * KVL_MLA_NO_FUSED_PROJECTION=1 sets 0 at initialisation. */
int kvl_mla_set_fused_projection(int on);
/* Extension, no counterpart in the reference, for tests of the failure path: the bound of every
 * device wait of the fused form above, in ticks of the GPU's 100 MHz real-time counter (0
 * restores the default, 2,000,000 = 20 ms). A wait that reaches it ends, the launch runs to its
 * end with invalid results, and the call reports it (a host-buffer call returns -1, a
 * stream-ordered one through kvl_mla_synchronize); the next call clears the device flags and
 * computes normally. Returns 0, or -1. */
int kvl_mla_set_fused_wait_limit(unsigned ticks);
int kvl_mla_timing_stages(unsigned mask);
int kvl_mla_timing_read(double *ms, int *count);
void *kvl_mla_event_record(void);
double kvl_mla_event_elapsed_ms(void *start, void *end);
int kvl_mla_event_destroy(void *event);
int kvl_mla_copy_kernel(void *dst, const void *src, size_t bytes);
/* A streaming read of bytes (% 16 == 0) from a 16-byte aligned device buffer, enqueued on
 * kvl_mla_stream(): the measured read-bandwidth ceiling beside the nominal HBM peak. */
int kvl_mla_read_kernel(const void *src, size_t bytes);
/* An empty kernel (256 workgroups of 1024 threads that do nothing), enqueued on
 * kvl_mla_stream(): captured back to back in a graph, it measures the per-launch cost of a
 * kernel boundary, the fixed cost every stage of a decode step pays. */
int kvl_mla_empty_kernel(void);

/* Quantiser boundary, computed on the GPU: for row i, latent [n, R] (already normalised) ->
 * int8 codes [n, R] + fp32 scale [n]; k_rope_raw [n, DR] (before rotation) -> RoPE at
 * positions[i] -> BF16 RNE [n, DR]. Same rows as src/mla_compressed_q8_state.c:34-55,
 * 121-125 produce from the same fp32 latent. */
int kvl_mla_q8_pack_rows(int8_t *codes, float *scales, uint16_t *rope_bf16, const float *latent,
                         const float *k_rope_raw, const int *positions, int n, int R, int DR,
                         float theta);

/* Synthetic histories generated on the device (benchmarks): rows [row0, row0 + nrows) of the
 * state's device copy get latents ~ approx. N(0,1) (Irwin-Hall of four 24-bit uniforms from
 * SplitMix64(seed)), Q8-quantised (Q8 state) or rounded to BF16 (FP32 and BF16 states: one
 * seed gives both the same values). Sets len = row0 + nrows. The host arrays are only written
 * by the *_pull calls. */
int kvl_mla_compressed_q8_state_fill_synthetic(KvlMlaCompressedQ8State *state, int row0,
                                               int nrows, uint64_t seed);
int kvl_mla_compressed_state_fill_synthetic(KvlMlaCompressedState *state, int row0, int nrows,
                                            uint64_t seed);
int kvl_mla_compressed_q8_state_pull(KvlMlaCompressedQ8State *state, int row0, int nrows);
int kvl_mla_compressed_state_pull(KvlMlaCompressedState *state, int row0, int nrows);
int kvl_mla_compressed_bf16_state_fill_synthetic(KvlMlaCompressedBF16State *state, int row0, int nrows,
                                                 uint64_t seed);
int kvl_mla_compressed_bf16_state_pull(KvlMlaCompressedBF16State *state, int row0, int nrows);

#ifdef __cplusplus
}
#endif

#endif
