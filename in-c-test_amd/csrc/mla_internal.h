// Internal interface between the host runtime (mla_runtime.cpp) and the HIP kernels
// (mla_decode.hip, mla_prefill.hip) of libkvl_mla. Not installed; the public C ABI is
// include/kvl/*.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kvl {

// Split-K partials one sequence may have (the combine kernels stage one weight per split).
constexpr int kMaxSplits = 2048;

// Sequences handled by one launch group. Per-sequence descriptors travel as kernel
// arguments (SeqTable, 64 x 48 B), so no per-call descriptor upload is needed.
constexpr int kMaxBatch = 64;

// Row formats of the latent history on the device.
enum Fmt : int {
    kFmtQ8 = 0,   // int8 codes [cap,R], fp32 scale [cap], bf16 RoPE key [cap,DR]
    kFmtF32 = 1,  // fp32 latent [cap,R], fp32 RoPE key [cap,DR]
    kFmtExp = 2,  // expanded fp32 keys [cap,NH,QD], values [cap,NH,DV]
    kFmtBF16 = 3, // bf16 latent [cap,R], bf16 RoPE key [cap,DR]
};

struct Dims {
    int H, NH, DN, DR, DV, R, QD, QO, KVO, KVB, HO;
};

// One sequence of a batched call. a/b/c are the device arrays of its history (see Fmt), pos
// the row appended by this step, len the number of rows attended (pos + 1). split0/nsplit
// locate its split-K partials; each split covers rps rows except the last, which takes the
// remainder.
struct SeqDesc {
    void *a;
    void *b;
    void *c;
    int len;
    int pos;
    int split0;
    int nsplit;
    int rps;
    int pad1;
};

struct SeqTable {
    SeqDesc s[kMaxBatch];
    int n;
};

// Device workspace of one decode launch group (all pointers device memory).
struct DecodeWork {
    float *x;        // [B,H]      input hidden states
    float *y;        // [ynp][B,QO+KVO] q_proj | kv_a outputs: ynp partials ypstride apart
    int ynp;         //            (their sum is the projection)
    size_t ypstride;
    float *qf;       // [B,NH,QS]  per-head score-space query (fp32)
    int8_t *qhi;     // [B,NH,R]   Q8 fast path: int8 query, high part
    int8_t *qlo;     // [B,NH,R]   Q8 fast path: int8 query, low part (x1/128)
    float *qs;       // [B,NH]     Q8 fast path: query dequant factor
    uint16_t *qrhi;  // [B,NH,DR]  Q8 fast path: RoPE query, bf16 high part
    uint16_t *qrlo;  // [B,NH,DR]  Q8 fast path: RoPE query, bf16 low part
    float *latent;   // [B,R]      expanded state: normalised latent of the new token
    float *kv;       // [B,KVB]    expanded state: kv_b expansion of the new token
    float *part;     // [splits, G, DVm+2] split-K partials (acc | m | l)
    float *scores;   // generic path: [P, G, Lmax] score scratch
    float *mix;      // [B*NH, DVm] normalised attention mix
    float *ho;       // [B,HO]     per-head outputs
    uint16_t *hos;   // [2][B,HO]  the same as bf16 hi | lo planes (compressed formats, R = 512)
    float *out;      // [B,H]      layer output
    uint8_t *rows;   // [B,row bytes] copy of the appended history rows (host write-back)
};

// ---- launchers (mla_decode.hip). All are stream-ordered and return hipError_t. ----

// Y[b, o] = (accumulate ? Y[b, o] : 0) + sum_i W[o, i] * X[b, i], for b < B. The output
// rows are the concatenation of W0 (out0 rows) and W1 (out1 rows, may be 0).
hipError_t launch_gemv(hipStream_t st, float *Y, int ldy, const float *X, int ldx, int B,
                       const uint16_t *W0, int out0, const uint16_t *W1, int out1, int in,
                       bool accumulate);

// Decode projection with the k range split over kGemvKs blocks: partial q of Y[b, o] at
// Y[q * pstride + b * ldy + o]; the consumer adds the partials in q order. Shapes accepted
// when gemv_ksplit_ok (in = 2048 or 4096; X and W 16-byte aligned), any B; otherwise
// hipErrorInvalidValue. A sequence's result does not depend on B or its place in the batch,
// so history rows appended by decode equal those the state prefill writes.
constexpr int kGemvKs = 4;
bool gemv_ksplit_ok(int in, int ldx);
// zero_flags (may be null): words kFqFlagStride * i and kFqFlagStride * i + 1, i < nzero, the
// launch clears (the readiness flags and combine counters of a fused Q8 attention launch that
// follows, FqArgs::flags).
hipError_t launch_gemv_ksplit(hipStream_t st, float *Y, size_t pstride, int ldy, const float *X,
                              int ldx, int B, const uint16_t *W0, int out0, const uint16_t *W1,
                              int out1, int in, unsigned *zero_flags = nullptr, int nzero = 0);
// The same kGemvKs partials (bit for bit) for S tokens given as bf16 planes XH, XL [S, in]
// (k_split's rounding), tiled over 128 tokens so a weight tile serves many of them: the
// prefill's kv_a projection and the state prefill. Shapes as launch_gemv_ksplit.
hipError_t launch_kva_tok(hipStream_t st, float *Y, size_t pstride, int ldy, const uint16_t *XH,
                          const uint16_t *XL, int S, const uint16_t *W, int out, int in);
// Y[b, o] (+)= sum_k W[o, k] x[b, k] with x given as bf16 planes XS[2][B][in] (hi, lo), as
// launch_combine writes them (DecodeWork::hos). Shapes when gemv_xs_ok (in = 2048 or 4096),
// any B.
bool gemv_xs_ok(int in);
// zf, nz (may be null): flag lines the launch clears (as launch_gemv_ksplit's zero_flags).
hipError_t launch_gemv_xs(hipStream_t st, float *Y, int ldy, const uint16_t *XS, int B,
                          const uint16_t *W, int out, int in, bool accumulate, unsigned *zf = nullptr,
                          int nz = 0);
// Clears the first 8 bytes of nlines flag lines (kFqFlagStride words apart).
hipError_t launch_clear_flags(hipStream_t st, unsigned *flags, int nlines);

// RMSNorm of katmp[b] (= y + koff) -> latent row; RoPE of katmp[b][R:] at s.pos. Writes the
// row into the history at row s.pos (fmt Q8/F32/BF16) or, for kFmtExp, the normalised latent
// into w.latent and the rotated key into the tail of w.rows. A copy of the stored row goes
// to w.rows for host write-back. rope_cs: [npos, DR/2] (cos, sin) pairs.
// nrows > 0: rows mode, nrows rows of the single sequence t.s[0] starting at t.s[0].pos,
// input row i at y + i*ldy, staged row i at w.rows + i*row_bytes.
// y holds ynp (1 or kGemvKs) partials ypstride floats apart; their in-order sum is the input.
hipError_t launch_append(hipStream_t st, int fmt, const SeqTable &t, const Dims &d,
                         const float *y, int ldy, int koff, int ynp, size_t ypstride,
                         const uint16_t *kv_a_norm, float eps, const float2 *rope_cs,
                         const DecodeWork &w, bool normed, int nrows);

// y[i] = RMSNorm(x[i]) * w for `rows` rows of length n (src/ops.c:76-83).
hipError_t launch_rmsnorm(hipStream_t st, float *y, const float *x, const uint16_t *w, int n,
                          int rows, float eps);

// Expanded state: scatter kv_b expansion + rotated key of the new token into keys/values.
hipError_t launch_store_expanded(hipStream_t st, const SeqTable &t, const Dims &d,
                                 const DecodeWork &w);

// Query preparation from w.y (w.ynp partials, w.ypstride apart): absorbed
// q_lat = W_UK^T q_nope and RoPE(q_rope) per head (fmt Q8/F32),
// or [q_nope | RoPE(q_rope)] (kFmtExp). quantize=true also builds the int8/bf16 split
// operands of the Q8 MFMA attention kernel.
hipError_t launch_qprep(hipStream_t st, int fmt, const SeqTable &t, const Dims &d,
                        const uint16_t *kv_b, const float2 *rope_cs, const DecodeWork &w,
                        bool quantize);
// launch_append (one row per sequence) and launch_qprep as one launch.
hipError_t launch_append_qprep(hipStream_t st, int fmt, const SeqTable &t, const Dims &d,
                               const float *y, int ldy, int koff, int ynp, size_t ypstride,
                               const uint16_t *kv_a_norm, float eps, const float2 *rope_cs,
                               const uint16_t *kv_b, const uint16_t *ukt, const DecodeWork &w, bool quantize);
// W_UK^T from kv_b (the first DN rows of each head) in the fragment order of the query
// preparation's MFMA operands (R = 512, DN = 128 only): ukt of launch_append_qprep.
hipError_t launch_wuk_transpose(hipStream_t st, uint16_t *dst, const uint16_t *kv_b, const Dims &d);

// Split-K attention over the history; writes partials (acc | m | l) per split.
// kind: 0 = generic VALU (any dims, one split per problem), 1 = FP32 rows as bf16 hi + lo on
// bf16 MFMA (Kimi dims), 2 = int8 MFMA (Kimi dims, Q8 rows), 3 = bf16 MFMA (Kimi dims, BF16 rows).
enum AttnKind : int { kAttnGeneric = 0, kAttnF32Mfma = 1, kAttnQ8Mfma = 2, kAttnBF16Mfma = 3 };
// members > 0: the sequences are the members of one block (tokens of one sequence, each with
// the split plan of its lone decode); the workgroups then go split-major, the members of a split
// together on one XCD, so that they share the history rows in its L2.
// What the Q8 attention launch needs to prepare the queries and append the rows itself (the
// work of launch_append_qprep, Kimi shapes): the q_proj | kv_a partials of launch_gemv_ksplit,
// W_UK^T in fragment order, the RoPE table, the kv_a norm weights, the caller's copy of the
// appended rows, the readiness flags (word kFqFlagStride * i; i in [0, B): query heads done,
// [kMaxBatch, kMaxBatch + B): row appended; zeroed by the launch_gemv_ksplit before it) and a
// host-visible word set when a wait for them timed out.
constexpr int kFqFlagStride = 32;  // FqArgs::flags: one 128-byte line per flag
struct FqArgs {
    float *y;  // written by the launch's projection tasks when gemv
    const uint16_t *ukt;
    const float2 *cs;
    const uint16_t *norm;
    uint8_t *rows;
    unsigned *flags;
    int *err;
    size_t pstride;
    int ldy, koff, row_bytes;
    float eps;
    // comb != 0: the launch also combines the split partials into ho / hos (launch_combine's
    // outputs, W_UV from kvb), split s of a sequence taking (head s / 2, half s % 2) and s + ns,
    // ... (flags words kFqFlagStride * (2 kMaxBatch + b), b < B, zeroed as the others).
    // comb = 1: every split of a sequence on one XCD, its partials read from that XCD's L2; needs
    // t.n a multiple of 8 and every sequence with the same split count ns, sequence b's splits
    // from b * ns (comb_ok). comb = 2: the partials stored past the L2s and read from memory;
    // needs 16 .. 255 splits per sequence (comb_cross_ok).
    int comb;
    const uint16_t *kvb;
    float *ho;
    uint16_t *hos;
    // gemv != 0: the launch also computes the q_proj | kv_a partials into y (k_gemv_ksplit's
    // blocks as tasks of its first kGemvTasks workgroups, the same arithmetic), from x [B, in]
    // (16-byte aligned rows, ldx) and the weights wq [out0, in], wkva [out1, in]; needs B <= 8
    // and in = 2048 (gemv_fuse_ok), and runs max(splits, kGemvTasks) workgroups. Flags words
    // kFqFlagStride * (3 kMaxBatch + i), i < kFqGemvFlags: per-head and kv_a task counts.
    int gemv;
    const float *x;
    const uint16_t *wq, *wkva;
    int ldx, in, out0, out1;
    int splits;  // the launch's split count (with gemv the grid is max(splits, kGemvTasks))
    unsigned spin;  // bound of every wait, in ticks of the 100 MHz real-time counter
};
constexpr unsigned kFqSpinTicks = 2000000;  // FqArgs::spin by default: 20 ms
// Lines of the flags buffer: query, row, combine (kMaxBatch each), then the projection counts
// (16 heads, kv_a). The o_proj launch after a fused launch clears them all (launch_gemv_xs's zf),
// and so does the q_proj | kv_a launch before one (launch_gemv_ksplit's zero_flags).
constexpr int kFqGemvFlags = 17;
constexpr int kFqFlagLines = 3 * kMaxBatch + kFqGemvFlags;
// Workgroups holding a projection task in the fused form: k_gemv_ksplit<1, 1>'s grid at the Kimi
// shapes (57 row blocks of 64 rows x 4 k quarters, blocks placed XCD-aware).
constexpr int kGemvTasks = 232;
// True when a fused launch with this table and split count can combine in place (FqArgs::comb).
bool comb_ok(const SeqTable &t, const Dims &d, int total_splits);
// True when a fused launch can also compute the q_proj | kv_a projection (FqArgs::gemv).
bool gemv_fuse_ok(const Dims &d, int B);
// True when a fused launch can combine across XCDs (FqArgs::comb = 2).
bool comb_cross_ok(const SeqTable &t, const Dims &d);
// fq: null, or the fused form (kind == kAttnQ8Mfma, members == 0, Kimi shapes, at most one
// round of workgroups, 17 B <= total_splits): blocks [0, 16 B) prepare one (sequence, head)
// query each, blocks [16 B, 17 B) append one row each, before their own split.
hipError_t launch_attention(hipStream_t st, int kind, int fmt, const SeqTable &t, const Dims &d,
                            int rows_per_split, int total_splits, int lmax,
                            const DecodeWork &w, int members = 0, const FqArgs *fq = nullptr);

// Normalise the split partials into mix[(b*G + g), DVm] and, for the compressed formats,
// apply W_UV: ho[b, h*DV + d] = sum_r kv_b[h*(DN+DV) + DN + d, r] * mix[b*NH + h, r].
// When combine_writes_hos(fmt, d), ho is also written to w.hos as bf16 hi | lo planes.
bool combine_writes_hos(int fmt, const Dims &d);
hipError_t launch_combine(hipStream_t st, int fmt, const SeqTable &t, const Dims &d,
                          const uint16_t *kv_b, const DecodeWork &w);

// Device-side generator of a synthetic Q8 / F32 / BF16 history (benchmark and test workloads):
// latents ~ Irwin-Hall(4) normal from SplitMix64, quantised with the history quantiser.
hipError_t launch_fill_history(hipStream_t st, int fmt, void *a, void *b, void *c, int R,
                               int DR, int row0, int nrows, uint64_t seed);

// Plain 16-byte vector copy (calibration of memory counters against known bytes).
hipError_t launch_copy(hipStream_t st, void *dst, const void *src, size_t bytes);
// Streaming read of `bytes` (a multiple of 16) by kReadBlocks x 256 threads; sink: device
// memory of kReadBlocks x 256 x 16 bytes (written only for one improbable bit pattern).
constexpr int kReadBlocks = 8192;
hipError_t launch_read(hipStream_t st, const void *src, size_t bytes, void *sink);
hipError_t launch_empty(hipStream_t st);

// ---- prefill (mla_prefill.hip) ----
// Device workspace bytes of a causal prefill of S tokens (generic: on the generic route).
size_t prefill_bytes(const Dims &d, int S, bool generic = false);
// Causal MLA prefill of S tokens: x [S,H] -> out [S,H] (device pointers), ws of
// prefill_bytes(d, S) bytes, rope_cs table covering positions [0, S).
// wo16: o_proj converted to fp16 (launch_bf16_to_f16), used by the MFMA route (the attention
// output enters the o_proj GEMM as fp16).
// kva (optional): asks for the kv_a projection of the S tokens in the decode arithmetic
// (launch_kva_tok partials, where prefill_kva_exact) so a state fill can reuse it; receives
// its place in ws, or kva->y = null when these dims do not allow it. Valid until ws is reused.
// Without kva the projection is part of the q GEMM (another summation order).
struct PrefillKva {
    const float *y;
    int ldy, np;
    size_t pstride;
};
// Range handling of the MFMA route (mla_prefill.hip): vscale (V) and oscale (the fp16 o_proj
// copy) are powers of two; sticky (optional) is raised with the call's own flag (the int after
// the first of ws: prefill_range_flag) when a query row falls outside the route's range.
// generic: take the generic route whatever the dims.
struct PrefillRange {
    float vscale = 1.0f, oscale = 1.0f;
    int *sticky = nullptr;
    bool generic = false;
};
// The per-call range flag of a prefill whose workspace is ws (MFMA route).
inline int *prefill_range_flag(void *ws) { return (int *)ws + 1; }
hipError_t launch_prefill_all(hipStream_t st, const Dims &d, int S, float eps, const float *x,
                              float *out, const uint16_t *wq, const uint16_t *wkva,
                              const uint16_t *wnorm, const uint16_t *wkvb, const uint16_t *wo,
                              const _Float16 *wo16, const float2 *rope_cs, void *ws,
                              PrefillKva *kva = nullptr, const PrefillRange *range = nullptr);
// True when a prefill of these dims can give its kv_a projection in the decode arithmetic.
bool prefill_kva_exact(const Dims &d);
// True when the prefill of these dims takes the MFMA route (needs the fp16 o_proj copy).
bool prefill_mfma_shape(const Dims &d);
// src [rows, cols] fp32 -> bf16 hi, lo planes (x = hi + lo to ~16 bits, both round to nearest
// even). cols % 8 == 0, 16-byte aligned rows.
hipError_t launch_split(hipStream_t st, const float *src, int ld_src, uint16_t *hi, uint16_t *lo,
                        int ld_dst, int rows, int cols);
// dst[i] = (fp16)(bf16 src[i] * scale), scale a power of two: exact while the scaled value is a
// normal fp16 (bf16 has 8 significant bits).
hipError_t launch_bf16_to_f16(hipStream_t st, _Float16 *dst, const uint16_t *src, size_t n, float scale);

}  // namespace kvl
