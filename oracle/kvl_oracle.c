/* CPU oracle of the MLA hot path -- TEST INFRASTRUCTURE ONLY (see kvl_oracle.h).
 *
 * Build without FP contraction or fast-math (the Makefile passes -ffp-contract=off): the
 * reference is compiled for x86-64 + AVX2 without FMA, so every product and sum below is a
 * separately rounded IEEE operation, exactly as there. */
#include "kvl_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_order = ORC_ORDER_AVX2;

void orc_set_order(int order) { g_order = order ? ORC_ORDER_AVX2 : ORC_ORDER_SCALAR; }
int orc_get_order(void) { return g_order; }

/* ---- bit helpers ------------------------------------------------------------------- */

/* src/ops.c:12-17: the BF16 word becomes the high half of the FP32 word. */
float orc_bf16_to_f32(uint16_t x) {
    const uint32_t bits = (uint32_t)x << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* src/mla_compressed_q8_state.c:9-16: round-to-nearest-even on the low 16 bits; values with
 * an all-ones exponent (Inf/NaN) are truncated, NaN payloads are not quietened. */
uint16_t orc_f32_to_bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, sizeof u);
    if ((u & 0x7f800000u) != 0x7f800000u) u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* ---- GEMV -------------------------------------------------------------------------- */

/* src/ops.c:19-24: double accumulation in index order, one rounding to float at the end. */
static float row_dot_scalar(const uint16_t *row, const float *x, int n) {
    double acc = 0.0;
    for (int i = 0; i < n; ++i) acc += (double)orc_bf16_to_f32(row[i]) * (double)x[i];
    return (float)acc;
}

/* src/ops.c:31-50: eight FP32 lanes, lane l owns indices i == l (mod 8) of the 8-aligned
 * body, each step is mul then add (no FMA). Lanes fold as (l0+l4, l1+l5, l2+l6, l3+l7), two
 * horizontal adds give (s0+s1)+(s2+s3), then the scalar tail is added in order. */
static float row_dot_avx2(const uint16_t *row, const float *x, int n) {
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) {
            const float p = orc_bf16_to_f32(row[i + l]) * x[i + l];
            lane[l] = lane[l] + p;
        }
    const float s0 = lane[0] + lane[4], s1 = lane[1] + lane[5];
    const float s2 = lane[2] + lane[6], s3 = lane[3] + lane[7];
    float r = (s0 + s1) + (s2 + s3);
    for (; i < n; ++i) {
        const float p = orc_bf16_to_f32(row[i]) * x[i];
        r = r + p;
    }
    return r;
}

/* src/ops.c:53-66 */
void orc_matvec_bf16(float *y, const float *x, const uint16_t *w, int in, int out) {
    const int avx2 = g_order == ORC_ORDER_AVX2;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; ++o) {
        const uint16_t *row = w + (size_t)o * (size_t)in;
        y[o] = avx2 ? row_dot_avx2(row, x, in) : row_dot_scalar(row, x, in);
    }
}

/* src/ops.c:76-83: mean square in double, inv = 1/sqrtf(float(ms/n)+eps), then (x*inv)*w. */
void orc_rmsnorm_bf16(float *y, const float *x, const uint16_t *weight, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float mean_sq = (float)(ss / (double)n);
    const float inv = 1.0f / sqrtf(mean_sq + eps);
    for (int i = 0; i < n; ++i) {
        const float t = x[i] * inv;
        y[i] = t * orc_bf16_to_f32(weight[i]);
    }
}

/* src/mla_compressed_q8_state.c:18-32: pair i of the raw [e0,o0,e1,o1,...] projection rotates
 * by angle pos * theta^(-2i/dim) (double), cos/sin rounded to float; output is
 * [evens*c - odds*s | odds*c + evens*s]. */
void orc_rope_interleaved(float *dst, const float *raw, int dim, int position, float theta) {
    const int half = dim / 2;
    for (int i = 0; i < half; ++i) {
        const double freq = pow((double)theta, -((double)(2 * i) / (double)dim));
        const double ang = (double)position * freq;
        const float c = (float)cos(ang);
        const float s = (float)sin(ang);
        const float ev = raw[2 * i], od = raw[2 * i + 1];
        const float ec = ev * c, os = od * s, oc = od * c, es = ev * s;
        dst[i] = ec - os;
        dst[half + i] = oc + es;
    }
}

/* ---- Q8 row format ----------------------------------------------------------------- */

/* src/mla_compressed_q8_state.c:34-55: symmetric absmax/127 with roundf (half away from
 * zero) on x * (1/scale); a zero or non-finite absmax gives zero codes and scale 1. */
void orc_quantize_latent(int8_t *dst, float *scale_out, const float *src, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(src[i]);
        if (a > amax) amax = a;
    }
    if (!(amax > 0.0f) || !isfinite(amax)) {
        memset(dst, 0, (size_t)n);
        *scale_out = 1.0f;
        return;
    }
    const float scale = amax / 127.0f;
    const float inv = 1.0f / scale;
    for (int i = 0; i < n; ++i) {
        float q = roundf(src[i] * inv);
        q = q > 127.0f ? 127.0f : q;
        q = q < -127.0f ? -127.0f : q;
        dst[i] = (int8_t)q;
    }
    *scale_out = scale;
}

/* src/mla_compressed_q8_state.c:57-61 */
float orc_dequant(int8_t q, float scale) { return (float)q * scale; }

void orc_q8_pack_row(int8_t *codes, float *scale, uint16_t *rope_bf16, const float *latent,
                     const float *k_rope_raw, int R, int DR, int position, float theta) {
    float *rot = (float *)malloc((size_t)DR * sizeof(float));
    orc_quantize_latent(codes, scale, latent, R);
    if (!rot) return;
    orc_rope_interleaved(rot, k_rope_raw, DR, position, theta);
    for (int d = 0; d < DR; ++d) rope_bf16[d] = orc_f32_to_bf16_rne(rot[d]);
    free(rot);
}

/* src/mla_compressed_q8_state.c:119-125 after the kv_a GEMV. */
void orc_q8_row_from_katmp(int8_t *codes, float *scale, uint16_t *rope_bf16, const float *katmp,
                           const uint16_t *kv_a_norm, int R, int DR, float eps, int position,
                           float theta) {
    float *lat = (float *)malloc((size_t)R * sizeof(float));
    if (!lat) return;
    orc_rmsnorm_bf16(lat, katmp, kv_a_norm, R, eps);
    orc_q8_pack_row(codes, scale, rope_bf16, lat, katmp + R, R, DR, position, theta);
    free(lat);
}

/* ---- shared checks ------------------------------------------------------------------ */

typedef struct {
    int H, NH, DN, DR, DV, R, QD, QO, KVO, KVB, HO;
} Dims;

static int dims_of(const KvlMlaConfig *cfg, Dims *d) {
    if (!cfg || cfg->hidden_size <= 0 || cfg->num_heads <= 0 || cfg->qk_nope_dim <= 0 ||
        cfg->qk_rope_dim <= 0 || (cfg->qk_rope_dim & 1) || cfg->v_head_dim <= 0 ||
        cfg->kv_lora_rank <= 0 || !(cfg->rope_theta > 0.0f))
        return -1;
    d->H = cfg->hidden_size;
    d->NH = cfg->num_heads;
    d->DN = cfg->qk_nope_dim;
    d->DR = cfg->qk_rope_dim;
    d->DV = cfg->v_head_dim;
    d->R = cfg->kv_lora_rank;
    d->QD = d->DN + d->DR;
    d->QO = d->NH * d->QD;
    d->KVO = d->R + d->DR;
    d->KVB = d->NH * (d->DN + d->DV);
    d->HO = d->NH * d->DV;
    return 0;
}

static int weights_ok(const KvlMlaBF16 *w) {
    return w && w->q_proj && w->kv_a_proj && w->kv_a_norm && w->kv_b_proj && w->o_proj;
}

/* ---- absorbed attention over a latent history ----------------------------------------
 * src/mla_compressed_state.c:118-157 and src/mla_compressed_q8_state.c:201-248 share one
 * arithmetic: per head, q_lat[r] = sum_d kv_b[h*(DN+DV)+d, r] * q_nope[d] (double);
 * score_j = float(sum_r q_lat*lat_j + sum_d q_rope*rope_j) * scale with ONE double
 * accumulator; p_j = expf(score_j - max) in float, denom in double; mix[r] =
 * sum_j (p_j/denom) * lat_j[r] (double, j ascending); out_h[d] = sum_r kv_b[..DN+d, r]*mix[r].
 * The history is handed over already widened to float rows (lat [L,R], rope [L,DR]). */
static void attend_latent(float *head_out, const float *qtmp, int position, const Dims *d,
                          const KvlMlaConfig *cfg, const uint16_t *kv_b, const float *lat,
                          const float *rope, float *qrope, float *q_lat, float *scores,
                          double *mixacc) {
    const int L = position + 1;
    const float scale = 1.0f / sqrtf((float)d->QD);
    for (int h = 0; h < d->NH; ++h) {
        const float *qh = qtmp + (size_t)h * d->QD;
        orc_rope_interleaved(qrope, qh + d->DN, d->DR, position, cfg->rope_theta);
        for (int r = 0; r < d->R; ++r) {
            double acc = 0.0;
            for (int k = 0; k < d->DN; ++k) {
                const size_t row = (size_t)h * (d->DN + d->DV) + (size_t)k;
                acc += (double)orc_bf16_to_f32(kv_b[row * d->R + r]) * (double)qh[k];
            }
            q_lat[r] = (float)acc;
        }
        float mx = -INFINITY;
        for (int j = 0; j < L; ++j) {
            const float *lj = lat + (size_t)j * d->R;
            const float *rj = rope + (size_t)j * d->DR;
            double dot = 0.0;
            for (int r = 0; r < d->R; ++r) dot += (double)q_lat[r] * (double)lj[r];
            for (int k = 0; k < d->DR; ++k) dot += (double)qrope[k] * (double)rj[k];
            scores[j] = (float)dot * scale;
            if (scores[j] > mx) mx = scores[j];
        }
        double denom = 0.0;
        for (int j = 0; j < L; ++j) {
            scores[j] = expf(scores[j] - mx);
            denom += scores[j];
        }
        for (int r = 0; r < d->R; ++r) mixacc[r] = 0.0;
        for (int j = 0; j < L; ++j) {
            const double pj = (double)scores[j] / denom;
            const float *lj = lat + (size_t)j * d->R;
            for (int r = 0; r < d->R; ++r) mixacc[r] += pj * (double)lj[r];
        }
        float *ho = head_out + (size_t)h * d->DV;
        for (int k = 0; k < d->DV; ++k) {
            const size_t row = (size_t)h * (d->DN + d->DV) + (size_t)d->DN + (size_t)k;
            double acc = 0.0;
            for (int r = 0; r < d->R; ++r)
                acc += (double)orc_bf16_to_f32(kv_b[row * d->R + r]) * (double)(float)mixacc[r];
            ho[k] = (float)acc;
        }
    }
}

/* ---- expanded state (src/mla_state.c) ------------------------------------------------ */

int orc_mla_state_init(KvlMlaState *s, const KvlMlaConfig *cfg, int capacity) {
    if (!s || !cfg || capacity <= 0 || cfg->num_heads <= 0 || cfg->qk_nope_dim <= 0 ||
        cfg->qk_rope_dim <= 0 || cfg->v_head_dim <= 0)
        return -1;
    memset(s, 0, sizeof(*s));
    const size_t qd = (size_t)cfg->qk_nope_dim + (size_t)cfg->qk_rope_dim;
    s->keys = (float *)calloc((size_t)capacity * (size_t)cfg->num_heads * qd, sizeof(float));
    s->values = (float *)calloc((size_t)capacity * (size_t)cfg->num_heads * (size_t)cfg->v_head_dim,
                                sizeof(float));
    if (!s->keys || !s->values) {
        orc_mla_state_free(s);
        return -1;
    }
    s->capacity = capacity;
    s->num_heads = cfg->num_heads;
    s->qk_nope_dim = cfg->qk_nope_dim;
    s->qk_rope_dim = cfg->qk_rope_dim;
    s->v_head_dim = cfg->v_head_dim;
    return 0;
}

void orc_mla_state_reset(KvlMlaState *s) {
    if (s) s->len = 0;
}

void orc_mla_state_free(KvlMlaState *s) {
    if (!s) return;
    free(s->keys);
    free(s->values);
    memset(s, 0, sizeof(*s));
}

size_t orc_mla_state_bytes(const KvlMlaState *s) {
    if (!s || s->capacity <= 0) return 0;
    const size_t qd = (size_t)s->qk_nope_dim + (size_t)s->qk_rope_dim;
    const size_t per = (size_t)s->num_heads * (qd + (size_t)s->v_head_dim) * sizeof(float);
    return sizeof(*s) + (size_t)s->capacity * per;
}

/* src/mla_state.c:66-149: expand the current token through kv_b, store K=[k_nope|rope] and V
 * per head, then attend with one double dot over QD. */
int orc_mla_decode_bf16(float *out, const float *x, int position, const KvlMlaConfig *cfg,
                        const KvlMlaBF16 *w, KvlMlaState *s) {
    Dims d;
    if (!out || !x || !cfg || !weights_ok(w) || !s || position != s->len || position < 0 ||
        position >= s->capacity || s->num_heads != cfg->num_heads ||
        s->qk_nope_dim != cfg->qk_nope_dim || s->qk_rope_dim != cfg->qk_rope_dim ||
        s->v_head_dim != cfg->v_head_dim || dims_of(cfg, &d) != 0)
        return -1;
    float *qtmp = (float *)malloc((size_t)d.QO * sizeof(float));
    float *katmp = (float *)malloc((size_t)d.KVO * sizeof(float));
    float *latent = (float *)malloc((size_t)d.R * sizeof(float));
    float *kvtmp = (float *)malloc((size_t)d.KVB * sizeof(float));
    float *rope = (float *)malloc((size_t)d.DR * sizeof(float));
    float *q = (float *)malloc((size_t)d.QD * sizeof(float));
    float *ho = (float *)malloc((size_t)d.HO * sizeof(float));
    float *scores = (float *)malloc((size_t)(position + 1) * sizeof(float));
    int rc = -1;
    if (!qtmp || !katmp || !latent || !kvtmp || !rope || !q || !ho || !scores) goto done;

    orc_matvec_bf16(qtmp, x, w->q_proj, d.H, d.QO);
    orc_matvec_bf16(katmp, x, w->kv_a_proj, d.H, d.KVO);
    orc_rmsnorm_bf16(latent, katmp, w->kv_a_norm, d.R, cfg->rms_eps);
    orc_matvec_bf16(kvtmp, latent, w->kv_b_proj, d.R, d.KVB);
    orc_rope_interleaved(rope, katmp + d.R, d.DR, position, cfg->rope_theta);

    const float scale = 1.0f / sqrtf((float)d.QD);
    for (int h = 0; h < d.NH; ++h) {
        const float *qh = qtmp + (size_t)h * d.QD;
        memcpy(q, qh, (size_t)d.DN * sizeof(float));
        orc_rope_interleaved(q + d.DN, qh + d.DN, d.DR, position, cfg->rope_theta);
        const float *kvh = kvtmp + (size_t)h * (d.DN + d.DV);
        float *kc = s->keys + ((size_t)position * d.NH + h) * d.QD;
        float *vc = s->values + ((size_t)position * d.NH + h) * d.DV;
        memcpy(kc, kvh, (size_t)d.DN * sizeof(float));
        memcpy(kc + d.DN, rope, (size_t)d.DR * sizeof(float));
        memcpy(vc, kvh + d.DN, (size_t)d.DV * sizeof(float));

        float mx = -INFINITY;
        for (int j = 0; j <= position; ++j) {
            const float *kj = s->keys + ((size_t)j * d.NH + h) * d.QD;
            double dot = 0.0;
            for (int k = 0; k < d.QD; ++k) dot += (double)q[k] * (double)kj[k];
            scores[j] = (float)dot * scale;
            if (scores[j] > mx) mx = scores[j];
        }
        double denom = 0.0;
        for (int j = 0; j <= position; ++j) {
            scores[j] = expf(scores[j] - mx);
            denom += scores[j];
        }
        for (int k = 0; k < d.DV; ++k) {
            double acc = 0.0;
            for (int j = 0; j <= position; ++j)
                acc += ((double)scores[j] / denom) *
                       (double)s->values[((size_t)j * d.NH + h) * d.DV + k];
            ho[(size_t)h * d.DV + k] = (float)acc;
        }
    }
    orc_matvec_bf16(out, ho, w->o_proj, d.HO, d.H);
    s->len = position + 1;
    rc = 0;
done:
    free(qtmp); free(katmp); free(latent); free(kvtmp); free(rope); free(q); free(ho);
    free(scores);
    return rc;
}

/* ---- compressed FP32 state (src/mla_compressed_state.c) ------------------------------ */

int orc_mla_compressed_state_init(KvlMlaCompressedState *s, const KvlMlaConfig *cfg, int capacity) {
    if (!s || !cfg || capacity <= 0 || cfg->kv_lora_rank <= 0 || cfg->qk_rope_dim <= 0 ||
        (cfg->qk_rope_dim & 1))
        return -1;
    memset(s, 0, sizeof(*s));
    s->latent = (float *)calloc((size_t)capacity * cfg->kv_lora_rank, sizeof(float));
    s->rope = (float *)calloc((size_t)capacity * cfg->qk_rope_dim, sizeof(float));
    if (!s->latent || !s->rope) {
        orc_mla_compressed_state_free(s);
        return -1;
    }
    s->capacity = capacity;
    s->kv_lora_rank = cfg->kv_lora_rank;
    s->qk_rope_dim = cfg->qk_rope_dim;
    return 0;
}

void orc_mla_compressed_state_reset(KvlMlaCompressedState *s) {
    if (s) s->len = 0;
}

int orc_mla_compressed_state_truncate(KvlMlaCompressedState *s, int new_len) {
    if (!s || new_len < 0 || new_len > s->len) return -1;
    s->len = new_len;
    return 0;
}

void orc_mla_compressed_state_free(KvlMlaCompressedState *s) {
    if (!s) return;
    free(s->latent);
    free(s->rope);
    memset(s, 0, sizeof(*s));
}

size_t orc_mla_compressed_state_bytes(const KvlMlaCompressedState *s) {
    if (!s || s->capacity <= 0) return 0;
    return sizeof(*s) +
           (size_t)s->capacity * ((size_t)s->kv_lora_rank + (size_t)s->qk_rope_dim) * sizeof(float);
}

/* src/mla_compressed_state.c:52-84 */
int orc_mla_compressed_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                          const KvlMlaBF16 *w, KvlMlaCompressedState *s) {
    if (!x || !cfg || !w || !s || !w->kv_a_proj || !w->kv_a_norm || seq_len <= 0 || s->len != 0 ||
        seq_len > s->capacity || s->kv_lora_rank != cfg->kv_lora_rank ||
        s->qk_rope_dim != cfg->qk_rope_dim)
        return -1;
    const int H = cfg->hidden_size, R = cfg->kv_lora_rank, DR = cfg->qk_rope_dim;
    if (H <= 0 || R <= 0 || DR <= 0 || (DR & 1) || !(cfg->rope_theta > 0.0f)) return -1;
    float *katmp = (float *)malloc((size_t)(R + DR) * sizeof(float));
    if (!katmp) return -1;
    for (int t = 0; t < seq_len; ++t) {
        orc_matvec_bf16(katmp, x + (size_t)t * H, w->kv_a_proj, H, R + DR);
        orc_rmsnorm_bf16(s->latent + (size_t)t * R, katmp, w->kv_a_norm, R, cfg->rms_eps);
        orc_rope_interleaved(s->rope + (size_t)t * DR, katmp + R, DR, t, cfg->rope_theta);
    }
    s->len = seq_len;
    free(katmp);
    return 0;
}

/* src/mla_compressed_state.c:86-161 */
int orc_mla_decode_compressed_bf16(float *out, const float *x, int position,
                                   const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                   KvlMlaCompressedState *s) {
    Dims d;
    if (!out || !x || !cfg || !weights_ok(w) || !s || position != s->len || position < 0 ||
        position >= s->capacity || s->kv_lora_rank != cfg->kv_lora_rank ||
        s->qk_rope_dim != cfg->qk_rope_dim || dims_of(cfg, &d) != 0)
        return -1;
    float *qtmp = (float *)malloc((size_t)d.QO * sizeof(float));
    float *katmp = (float *)malloc((size_t)d.KVO * sizeof(float));
    float *qrope = (float *)malloc((size_t)d.DR * sizeof(float));
    float *q_lat = (float *)malloc((size_t)d.R * sizeof(float));
    double *mixacc = (double *)malloc((size_t)d.R * sizeof(double));
    float *scores = (float *)malloc((size_t)(position + 1) * sizeof(float));
    float *ho = (float *)malloc((size_t)d.HO * sizeof(float));
    int rc = -1;
    if (!qtmp || !katmp || !qrope || !q_lat || !mixacc || !scores || !ho) goto done;

    orc_matvec_bf16(qtmp, x, w->q_proj, d.H, d.QO);
    orc_matvec_bf16(katmp, x, w->kv_a_proj, d.H, d.KVO);
    orc_rmsnorm_bf16(s->latent + (size_t)position * d.R, katmp, w->kv_a_norm, d.R, cfg->rms_eps);
    orc_rope_interleaved(s->rope + (size_t)position * d.DR, katmp + d.R, d.DR, position,
                         cfg->rope_theta);
    attend_latent(ho, qtmp, position, &d, cfg, w->kv_b_proj, s->latent, s->rope, qrope, q_lat,
                  scores, mixacc);
    orc_matvec_bf16(out, ho, w->o_proj, d.HO, d.H);
    s->len = position + 1;
    rc = 0;
done:
    free(qtmp); free(katmp); free(qrope); free(q_lat); free(mixacc); free(scores); free(ho);
    return rc;
}

/* The library's BF16-latent history (an extension with no function of its own in the reference):
 * the FP32 decode above, src/mla_compressed_state.c:86-161, with the appended latent row and
 * rotated key rounded to bf16 (src/mla_compressed_q8_state.c:9-16, orc_f32_to_bf16_rne) before
 * they are stored and attended. Over an FP32 state whose earlier rows are bf16 values, this is
 * what the library's BF16 state computes: its rows, widened to fp32, are these rows. */
int orc_mla_decode_compressed_bf16_rows(float *out, const float *x, int position,
                                        const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                        KvlMlaCompressedState *s) {
    Dims d;
    if (!out || !x || !cfg || !weights_ok(w) || !s || position != s->len || position < 0 ||
        position >= s->capacity || s->kv_lora_rank != cfg->kv_lora_rank ||
        s->qk_rope_dim != cfg->qk_rope_dim || dims_of(cfg, &d) != 0)
        return -1;
    float *qtmp = (float *)malloc((size_t)d.QO * sizeof(float));
    float *katmp = (float *)malloc((size_t)d.KVO * sizeof(float));
    float *qrope = (float *)malloc((size_t)d.DR * sizeof(float));
    float *q_lat = (float *)malloc((size_t)d.R * sizeof(float));
    double *mixacc = (double *)malloc((size_t)d.R * sizeof(double));
    float *scores = (float *)malloc((size_t)(position + 1) * sizeof(float));
    float *ho = (float *)malloc((size_t)d.HO * sizeof(float));
    int rc = -1;
    if (!qtmp || !katmp || !qrope || !q_lat || !mixacc || !scores || !ho) goto done;

    orc_matvec_bf16(qtmp, x, w->q_proj, d.H, d.QO);
    orc_matvec_bf16(katmp, x, w->kv_a_proj, d.H, d.KVO);
    float *lat = s->latent + (size_t)position * d.R, *rope = s->rope + (size_t)position * d.DR;
    orc_rmsnorm_bf16(lat, katmp, w->kv_a_norm, d.R, cfg->rms_eps);
    orc_rope_interleaved(rope, katmp + d.R, d.DR, position, cfg->rope_theta);
    for (int r = 0; r < d.R; ++r) lat[r] = orc_bf16_to_f32(orc_f32_to_bf16_rne(lat[r]));
    for (int k = 0; k < d.DR; ++k) rope[k] = orc_bf16_to_f32(orc_f32_to_bf16_rne(rope[k]));
    attend_latent(ho, qtmp, position, &d, cfg, w->kv_b_proj, s->latent, s->rope, qrope, q_lat,
                  scores, mixacc);
    orc_matvec_bf16(out, ho, w->o_proj, d.HO, d.H);
    s->len = position + 1;
    rc = 0;
done:
    free(qtmp); free(katmp); free(qrope); free(q_lat); free(mixacc); free(scores); free(ho);
    return rc;
}

/* src/mla_compressed_state.c:163-184 */
int orc_mla_decode_compressed_block_bf16(float *out, const float *x, int count, int start_position,
                                         const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                         KvlMlaCompressedState *s) {
    if (!out || !x || !cfg || !w || !s || count <= 0 || start_position != s->len ||
        start_position < 0 || count > s->capacity - start_position)
        return -1;
    const int H = cfg->hidden_size;
    if (H <= 0) return -1;
    for (int t = 0; t < count; ++t)
        if (orc_mla_decode_compressed_bf16(out + (size_t)t * H, x + (size_t)t * H,
                                           start_position + t, cfg, w, s) != 0)
            return -1;
    return 0;
}

/* ---- compressed Q8 state (src/mla_compressed_q8_state.c) ----------------------------- */

int orc_mla_compressed_q8_state_init(KvlMlaCompressedQ8State *s, const KvlMlaConfig *cfg,
                                     int capacity) {
    if (!s || !cfg || capacity <= 0 || cfg->kv_lora_rank <= 0 || cfg->qk_rope_dim <= 0 ||
        (cfg->qk_rope_dim & 1))
        return -1;
    memset(s, 0, sizeof(*s));
    s->latent_q8 = (int8_t *)calloc((size_t)capacity * cfg->kv_lora_rank, 1);
    s->latent_scale = (float *)calloc((size_t)capacity, sizeof(float));
    s->rope_bf16 = (uint16_t *)calloc((size_t)capacity * cfg->qk_rope_dim, sizeof(uint16_t));
    if (!s->latent_q8 || !s->latent_scale || !s->rope_bf16) {
        orc_mla_compressed_q8_state_free(s);
        return -1;
    }
    s->capacity = capacity;
    s->kv_lora_rank = cfg->kv_lora_rank;
    s->qk_rope_dim = cfg->qk_rope_dim;
    return 0;
}

void orc_mla_compressed_q8_state_reset(KvlMlaCompressedQ8State *s) {
    if (s) s->len = 0;
}

int orc_mla_compressed_q8_state_truncate(KvlMlaCompressedQ8State *s, int new_len) {
    if (!s || new_len < 0 || new_len > s->len) return -1;
    s->len = new_len;
    return 0;
}

void orc_mla_compressed_q8_state_free(KvlMlaCompressedQ8State *s) {
    if (!s) return;
    free(s->latent_q8);
    free(s->latent_scale);
    free(s->rope_bf16);
    memset(s, 0, sizeof(*s));
}

size_t orc_mla_compressed_q8_state_bytes(const KvlMlaCompressedQ8State *s) {
    if (!s || s->capacity <= 0) return 0;
    return sizeof(*s) + (size_t)s->capacity * ((size_t)s->kv_lora_rank + sizeof(float) +
                                               (size_t)s->qk_rope_dim * sizeof(uint16_t));
}

/* src/mla_compressed_q8_state.c:111-127 */
static void q8_append(const float *x, int position, const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                      KvlMlaCompressedQ8State *s, float *katmp) {
    const int H = cfg->hidden_size, R = cfg->kv_lora_rank, DR = cfg->qk_rope_dim;
    orc_matvec_bf16(katmp, x, w->kv_a_proj, H, R + DR);
    orc_q8_row_from_katmp(s->latent_q8 + (size_t)position * R, s->latent_scale + position,
                          s->rope_bf16 + (size_t)position * DR, katmp, w->kv_a_norm, R, DR,
                          cfg->rms_eps, position, cfg->rope_theta);
}

/* src/mla_compressed_q8_state.c:129-159 */
int orc_mla_compressed_q8_state_prefill_bf16(const float *x, int seq_len, const KvlMlaConfig *cfg,
                                             const KvlMlaBF16 *w, KvlMlaCompressedQ8State *s) {
    if (!x || !cfg || !w || !s || !w->kv_a_proj || !w->kv_a_norm || seq_len <= 0 || s->len != 0 ||
        seq_len > s->capacity || s->kv_lora_rank != cfg->kv_lora_rank ||
        s->qk_rope_dim != cfg->qk_rope_dim)
        return -1;
    const int H = cfg->hidden_size, R = cfg->kv_lora_rank, DR = cfg->qk_rope_dim;
    if (H <= 0 || R <= 0 || DR <= 0 || (DR & 1) || !(cfg->rope_theta > 0.0f)) return -1;
    float *katmp = (float *)malloc((size_t)(R + DR) * sizeof(float));
    if (!katmp) return -1;
    for (int t = 0; t < seq_len; ++t) q8_append(x + (size_t)t * H, t, cfg, w, s, katmp);
    s->len = seq_len;
    free(katmp);
    return 0;
}

/* src/mla_compressed_q8_state.c:161-255: the Q8 history is read through dequant_latent
 * ((float)q * scale) and the BF16 RoPE keys widened to float; the arithmetic is then the
 * FP32 decode's. */
int orc_mla_decode_compressed_q8_bf16(float *out, const float *x, int position,
                                      const KvlMlaConfig *cfg, const KvlMlaBF16 *w,
                                      KvlMlaCompressedQ8State *s) {
    Dims d;
    if (!out || !x || !cfg || !weights_ok(w) || !s || position != s->len || position < 0 ||
        position >= s->capacity || s->kv_lora_rank != cfg->kv_lora_rank ||
        s->qk_rope_dim != cfg->qk_rope_dim || dims_of(cfg, &d) != 0)
        return -1;
    const int L = position + 1;
    float *qtmp = (float *)malloc((size_t)d.QO * sizeof(float));
    float *katmp = (float *)malloc((size_t)d.KVO * sizeof(float));
    float *qrope = (float *)malloc((size_t)d.DR * sizeof(float));
    float *q_lat = (float *)malloc((size_t)d.R * sizeof(float));
    double *mixacc = (double *)malloc((size_t)d.R * sizeof(double));
    float *scores = (float *)malloc((size_t)L * sizeof(float));
    float *ho = (float *)malloc((size_t)d.HO * sizeof(float));
    float *lat = (float *)malloc((size_t)L * d.R * sizeof(float));
    float *rope = (float *)malloc((size_t)L * d.DR * sizeof(float));
    int rc = -1;
    if (!qtmp || !katmp || !qrope || !q_lat || !mixacc || !scores || !ho || !lat || !rope) goto done;

    orc_matvec_bf16(qtmp, x, w->q_proj, d.H, d.QO);
    q8_append(x, position, cfg, w, s, katmp);
    for (int j = 0; j < L; ++j) {
        for (int r = 0; r < d.R; ++r)
            lat[(size_t)j * d.R + r] =
                orc_dequant(s->latent_q8[(size_t)j * d.R + r], s->latent_scale[j]);
        for (int k = 0; k < d.DR; ++k)
            rope[(size_t)j * d.DR + k] = orc_bf16_to_f32(s->rope_bf16[(size_t)j * d.DR + k]);
    }
    attend_latent(ho, qtmp, position, &d, cfg, w->kv_b_proj, lat, rope, qrope, q_lat, scores,
                  mixacc);
    orc_matvec_bf16(out, ho, w->o_proj, d.HO, d.H);
    s->len = position + 1;
    rc = 0;
done:
    free(qtmp); free(katmp); free(qrope); free(q_lat); free(mixacc); free(scores); free(ho);
    free(lat); free(rope);
    return rc;
}

/* ---- prefill ------------------------------------------------------------------------ */

/* src/mla_prefill_streaming.c:31-59 (dot_f32_f64). AVX2 order: two 4-lane double
 * accumulators over the 8-aligned body (elements 0-3 and 4-7 of each block), summed lane-wise,
 * folded as (l0+l1)+(l2+l3), then the tail in order. */
static double dot_f64(const float *a, const float *b, int n) {
    if (g_order == ORC_ORDER_AVX2) {
        double a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
        int i = 0;
        for (; i + 8 <= n; i += 8)
            for (int l = 0; l < 4; ++l) {
                const double p0 = (double)a[i + l] * (double)b[i + l];
                const double p1 = (double)a[i + 4 + l] * (double)b[i + 4 + l];
                a0[l] = a0[l] + p0;
                a1[l] = a1[l] + p1;
            }
        double lane[4];
        for (int l = 0; l < 4; ++l) lane[l] = a0[l] + a1[l];
        double acc = (lane[0] + lane[1]) + (lane[2] + lane[3]);
        for (; i < n; ++i) acc += (double)a[i] * (double)b[i];
        return acc;
    }
    double acc = 0.0;
    for (int i = 0; i < n; ++i) acc += (double)a[i] * (double)b[i];
    return acc;
}

/* src/mla_prefill_streaming.c:78-206 */
/* Query rows of the streaming prefill: all S rows (rows == NULL; out [S, H], heads written to
 * out as the reference does when HO == H), or the listed rows only (out [nrows, H]: row i of
 * out is query row rows[i]). A listed row takes exactly the arithmetic of the full form (its
 * kv_a, keys and values of every j <= t, its query, scores, softmax and o_proj), so it equals
 * that row of the full prefill bit for bit. */
static int prefill_streaming_rows(float *out, const float *x, int seq_len, const int *rows,
                                  int nrows, const KvlMlaConfig *cfg, const KvlMlaBF16 *w) {
    Dims d;
    if (!out || !x || !cfg || !weights_ok(w) || seq_len <= 0 || dims_of(cfg, &d) != 0) return -1;
    int S = seq_len;
    const int KHV = d.DN + d.DV;
    const int NQ = rows ? nrows : S;
    if (rows) {
        if (nrows <= 0) return -1;
        int last = 0;
        for (int i = 0; i < nrows; ++i) {
            if (rows[i] < 0 || rows[i] >= seq_len) return -1;
            if (rows[i] > last) last = rows[i];
        }
        S = last + 1; /* rows past the last query row are never attended */
    }
    int workers = 1;
#ifdef _OPENMP
    workers = omp_get_max_threads();
    if (workers < 1) workers = 1;
    if (workers > NQ) workers = NQ;
#endif
    float *lat = (float *)malloc((size_t)S * d.R * sizeof(float));
    float *rope = (float *)malloc((size_t)S * d.DR * sizeof(float));
    float *knope = (float *)malloc((size_t)S * d.DN * sizeof(float));
    float *vals = (float *)malloc((size_t)S * d.DV * sizeof(float));
    float *sc_all = (float *)malloc((size_t)workers * S * sizeof(float));
    float *q_all = (float *)malloc((size_t)workers * d.QD * sizeof(float));
    float *qr_all = (float *)malloc((size_t)workers * d.DR * sizeof(float));
    double *acc_all = (double *)malloc((size_t)workers * d.DV * sizeof(double));
    float *katmp = (float *)malloc((size_t)d.KVO * sizeof(float));
    float *kvtmp = (float *)malloc((size_t)KHV * sizeof(float));
    float *htmp = (float *)malloc((size_t)d.HO * sizeof(float));
    float *heads = (d.HO == d.H && !rows) ? out : (float *)malloc((size_t)NQ * d.HO * sizeof(float));
    int rc = -1;
    if (!lat || !rope || !knope || !vals || !sc_all || !q_all || !qr_all || !acc_all || !katmp ||
        !kvtmp || !htmp || !heads)
        goto done;

    for (int t = 0; t < S; ++t) {
        orc_matvec_bf16(katmp, x + (size_t)t * d.H, w->kv_a_proj, d.H, d.KVO);
        orc_rmsnorm_bf16(lat + (size_t)t * d.R, katmp, w->kv_a_norm, d.R, cfg->rms_eps);
        orc_rope_interleaved(rope + (size_t)t * d.DR, katmp + d.R, d.DR, t, cfg->rope_theta);
    }
    const float scale = 1.0f / sqrtf((float)d.QD);
    for (int h = 0; h < d.NH; ++h) {
        const uint16_t *kvh = w->kv_b_proj + (size_t)h * KHV * d.R;
        for (int j = 0; j < S; ++j) {
            orc_matvec_bf16(kvtmp, lat + (size_t)j * d.R, kvh, d.R, KHV);
            memcpy(knope + (size_t)j * d.DN, kvtmp, (size_t)d.DN * sizeof(float));
            memcpy(vals + (size_t)j * d.DV, kvtmp + d.DN, (size_t)d.DV * sizeof(float));
        }
        const uint16_t *qh = w->q_proj + (size_t)h * d.QD * d.H;
        int i;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 8) if (NQ >= 128 || rows) num_threads(workers)
#endif
        for (i = 0; i < NQ; ++i) {
            const int t = rows ? rows[i] : i;
            int tid = 0;
#ifdef _OPENMP
            tid = omp_get_thread_num();
#endif
            float *sc = sc_all + (size_t)tid * S;
            float *q = q_all + (size_t)tid * d.QD;
            float *qr = qr_all + (size_t)tid * d.DR;
            double *acc = acc_all + (size_t)tid * d.DV;
            orc_matvec_bf16(q, x + (size_t)t * d.H, qh, d.H, d.QD);
            orc_rope_interleaved(qr, q + d.DN, d.DR, t, cfg->rope_theta);
            float mx = -INFINITY;
            for (int j = 0; j <= t; ++j) {
                const double dot = dot_f64(q, knope + (size_t)j * d.DN, d.DN) +
                                   dot_f64(qr, rope + (size_t)j * d.DR, d.DR);
                sc[j] = (float)dot * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double denom = 0.0;
            for (int j = 0; j <= t; ++j) {
                sc[j] = expf(sc[j] - mx);
                denom += sc[j];
            }
            for (int k = 0; k < d.DV; ++k) acc[k] = 0.0;
            for (int j = 0; j <= t; ++j) {
                const double p = (double)sc[j] / denom;
                const float *vj = vals + (size_t)j * d.DV;
                for (int k = 0; k < d.DV; ++k) {
                    const double pv = p * (double)vj[k];
                    acc[k] = acc[k] + pv;
                }
            }
            float *ho = heads + (size_t)i * d.HO + (size_t)h * d.DV;
            for (int k = 0; k < d.DV; ++k) ho[k] = (float)acc[k];
        }
    }
    for (int t = 0; t < NQ; ++t) {
        memcpy(htmp, heads + (size_t)t * d.HO, (size_t)d.HO * sizeof(float));
        orc_matvec_bf16(out + (size_t)t * d.H, htmp, w->o_proj, d.HO, d.H);
    }
    rc = 0;
done:
    free(lat); free(rope); free(knope); free(vals); free(sc_all); free(q_all); free(qr_all);
    free(acc_all); free(katmp); free(kvtmp); free(htmp);
    if (heads != out) free(heads);
    return rc;
}

int orc_mla_prefill_streaming(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg,
                              const KvlMlaBF16 *w) {
    return prefill_streaming_rows(out, x, seq_len, NULL, 0, cfg, w);
}

int orc_mla_prefill_streaming_rows(float *out, const float *x, int seq_len, const int *rows,
                                   int nrows, const KvlMlaConfig *cfg, const KvlMlaBF16 *w) {
    return prefill_streaming_rows(out, x, seq_len, rows, nrows, cfg, w);
}

/* src/ops.c:105-192: every token's Q, K=[k_nope|rope] and V materialised for all heads, then
 * causal attention with one double dot over QD and double PV. */
int orc_mla_prefill_materialized(float *out, const float *x, int seq_len, const KvlMlaConfig *cfg,
                                 const KvlMlaBF16 *w) {
    Dims d;
    if (!out || !x || !cfg || !weights_ok(w) || seq_len <= 0 || dims_of(cfg, &d) != 0) return -1;
    const int S = seq_len;
    float *qs = (float *)malloc((size_t)S * d.NH * d.QD * sizeof(float));
    float *ks = (float *)malloc((size_t)S * d.NH * d.QD * sizeof(float));
    float *vs = (float *)malloc((size_t)S * d.NH * d.DV * sizeof(float));
    float *qtmp = (float *)malloc((size_t)d.QO * sizeof(float));
    float *katmp = (float *)malloc((size_t)d.KVO * sizeof(float));
    float *latent = (float *)malloc((size_t)d.R * sizeof(float));
    float *kvtmp = (float *)malloc((size_t)d.KVB * sizeof(float));
    float *rope = (float *)malloc((size_t)d.DR * sizeof(float));
    float *ho = (float *)malloc((size_t)d.HO * sizeof(float));
    float *sc = (float *)malloc((size_t)S * sizeof(float));
    int rc = -1;
    if (!qs || !ks || !vs || !qtmp || !katmp || !latent || !kvtmp || !rope || !ho || !sc) goto done;

    for (int t = 0; t < S; ++t) {
        const float *xt = x + (size_t)t * d.H;
        orc_matvec_bf16(qtmp, xt, w->q_proj, d.H, d.QO);
        orc_matvec_bf16(katmp, xt, w->kv_a_proj, d.H, d.KVO);
        orc_rmsnorm_bf16(latent, katmp, w->kv_a_norm, d.R, cfg->rms_eps);
        orc_matvec_bf16(kvtmp, latent, w->kv_b_proj, d.R, d.KVB);
        orc_rope_interleaved(rope, katmp + d.R, d.DR, t, cfg->rope_theta);
        for (int h = 0; h < d.NH; ++h) {
            const float *qh = qtmp + (size_t)h * d.QD;
            float *qd = qs + ((size_t)t * d.NH + h) * d.QD;
            memcpy(qd, qh, (size_t)d.DN * sizeof(float));
            orc_rope_interleaved(qd + d.DN, qh + d.DN, d.DR, t, cfg->rope_theta);
            const float *kvh = kvtmp + (size_t)h * (d.DN + d.DV);
            float *kd = ks + ((size_t)t * d.NH + h) * d.QD;
            memcpy(kd, kvh, (size_t)d.DN * sizeof(float));
            memcpy(kd + d.DN, rope, (size_t)d.DR * sizeof(float));
            memcpy(vs + ((size_t)t * d.NH + h) * d.DV, kvh + d.DN, (size_t)d.DV * sizeof(float));
        }
    }
    const float scale = 1.0f / sqrtf((float)d.QD);
    for (int t = 0; t < S; ++t) {
        for (int h = 0; h < d.NH; ++h) {
            const float *q = qs + ((size_t)t * d.NH + h) * d.QD;
            float mx = -INFINITY;
            for (int j = 0; j <= t; ++j) {
                const float *k = ks + ((size_t)j * d.NH + h) * d.QD;
                double dot = 0.0;
                for (int i = 0; i < d.QD; ++i) dot += (double)q[i] * (double)k[i];
                sc[j] = (float)dot * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double denom = 0.0;
            for (int j = 0; j <= t; ++j) {
                sc[j] = expf(sc[j] - mx);
                denom += sc[j];
            }
            for (int k = 0; k < d.DV; ++k) {
                double acc = 0.0;
                for (int j = 0; j <= t; ++j)
                    acc += ((double)sc[j] / denom) * (double)vs[((size_t)j * d.NH + h) * d.DV + k];
                ho[(size_t)h * d.DV + k] = (float)acc;
            }
        }
        orc_matvec_bf16(out + (size_t)t * d.H, ho, w->o_proj, d.HO, d.H);
    }
    rc = 0;
done:
    free(qs); free(ks); free(vs); free(qtmp); free(katmp); free(latent); free(kvtmp); free(rope);
    free(ho); free(sc);
    return rc;
}
