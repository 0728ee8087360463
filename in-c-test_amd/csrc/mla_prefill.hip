// HIP kernels of the causal MLA prefill (src/mla_prefill_streaming.c:78-206 of the
// reference: non-absorbed attention, K/V expanded through kv_b for every token).
//
// MFMA route (H, R, QD multiples of 32, DV multiple of 16, DN multiple of 8):
//   split     x (fp32) -> bf16 hi + lo operands; a flag records whether any lo is non-zero
//   gemm      [q | kv_a] = x . W^T           (bf16 MFMA, fp32 accumulate, lo pass skipped
//                                             when the operand is exactly bf16)
//   kva_epi   RMSNorm -> latent (hi/lo), RoPE(k_rope) -> bf16, per token (RMSNorm as decode)
//   gemm      kv = latent . kv_b^T
//   pack      Q = [q_nope | RoPE(q_rope)] (hi/lo), K = [k_nope | k_rope] (bf16), V^T (bf16)
//   flash     causal attention per (64-query tile, head), online softmax, P as hi/lo bf16
//   gemm      out = heads . o_proj^T
// Generic route (any shape): the same stages with VALU kernels.
#include "mla_device.h"
#include "mla_internal.h"

#include <math.h>

namespace kvl {

// ================================================================ split ================

// src[r, c] (fp32, ld_src) -> hi/lo bf16 [rows, cols] (ld_dst); flag |= any lo != 0.
__global__ __launch_bounds__(256) void k_split(const float *src, int ld_src, uint16_t *hi,
                                               uint16_t *lo, int ld_dst, int rows, int cols,
                                               int *flag) {
    const size_t n = (size_t)rows * cols;
    int any = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t r = i / cols, c = i % cols;
        uint16_t h, l;
        split_bf16(src[r * ld_src + c], h, l);
        hi[r * ld_dst + c] = h;
        lo[r * ld_dst + c] = l;
        any |= (l & 0x7fff) != 0;
    }
    if (__syncthreads_or(any) && threadIdx.x == 0) atomicOr(flag, 1);
}

__global__ void k_zero_int(int *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// ================================================================ GEMM =================

// C[m, n] = sum_k (Ah + Al)[m, k] * B[n, k], all row-major, bf16 operands, fp32 output.
// Block tile 128 x 128, k step 32; wave (wm, wn) owns a 64 x 64 quadrant (4 x 4 MFMA tiles
// of v_mfma_f32_16x16x32_bf16). The lo operand pass runs when Al is given and either no
// flag is given or *lo_flag != 0 (the flag is raised by the producer of Al).
// Requires K % 32 == 0 and 16-byte aligned rows (lda, ldb multiples of 8).
constexpr int kGBm = 128, kGBn = 128, kGBk = 32, kGLd = 40;  // LDS row: 32 + 8 bf16

struct GemmArgs {
    const uint16_t *Ah, *Al, *B;
    float *C;
    const int *lo_flag;
    int M, N, K, lda, ldb, ldc;
};

__global__ __launch_bounds__(256) void k_gemm_bf16(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sah[kGBm * kGLd];
    __shared__ __attribute__((aligned(16))) uint16_t sal[kGBm * kGLd];
    __shared__ __attribute__((aligned(16))) uint16_t sb[kGBn * kGLd];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, n = l & 15, g = l >> 4;
    const int wm = w >> 1, wn = w & 1;
    const int m0 = blockIdx.y * kGBm, n0 = blockIdx.x * kGBn;
    const bool use_lo = a.Al && (!a.lo_flag || *a.lo_flag);
    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // each thread stages 2 x 16 B of A hi (and lo) and 2 x 16 B of B per k step
    v4i pa[2], pl[2], pb[2];
    auto load = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int p = tid + 256 * q, row = p >> 2, c8 = (p & 3) * 8;
            const int gm = m0 + row, gn = n0 + row;
            pa[q] = gm < a.M ? *(const v4i *)(a.Ah + (size_t)gm * a.lda + k0 + c8) : v4i{0, 0, 0, 0};
            if (use_lo)
                pl[q] = gm < a.M ? *(const v4i *)(a.Al + (size_t)gm * a.lda + k0 + c8) : v4i{0, 0, 0, 0};
            pb[q] = gn < a.N ? *(const v4i *)(a.B + (size_t)gn * a.ldb + k0 + c8) : v4i{0, 0, 0, 0};
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int p = tid + 256 * q, row = p >> 2, c8 = (p & 3) * 8;
            *(v4i *)(sah + row * kGLd + c8) = pa[q];
            if (use_lo) *(v4i *)(sal + row * kGLd + c8) = pl[q];
            *(v4i *)(sb + row * kGLd + c8) = pb[q];
        }
    };
    load(0);
    for (int k0 = 0; k0 < a.K; k0 += kGBk) {
        __syncthreads();
        stash();
        __syncthreads();
        if (k0 + kGBk < a.K) load(k0 + kGBk);
        v8bf bo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bo[j] = *(const v8bf *)(sb + (64 * wn + 16 * j + n) * kGLd + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const v8bf ah = *(const v8bf *)(sah + (64 * wm + 16 * i + n) * kGLd + 8 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma_bf16(ah, bo[j], acc[i][j]);
            if (use_lo) {
                const v8bf al = *(const v8bf *)(sal + (64 * wm + 16 * i + n) * kGLd + 8 * g);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma_bf16(al, bo[j], acc[i][j]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = n0 + 64 * wn + 16 * j + n;
            if (col >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + 64 * wm + 16 * i + 4 * g + r;
                if (row < a.M) a.C[(size_t)row * a.ldc + col] = acc[i][j][r];
            }
        }
}

static hipError_t gemm(hipStream_t st, const uint16_t *Ah, const uint16_t *Al, const int *flag,
                       int lda, const uint16_t *B, int ldb, float *C, int ldc, int M, int N,
                       int K) {
    GemmArgs a{Ah, Al, B, C, flag, M, N, K, lda, ldb, ldc};
    dim3 grid((N + kGBn - 1) / kGBn, (M + kGBm - 1) / kGBm);
    hipLaunchKernelGGL(k_gemm_bf16, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

// ================================================================ epilogues ============

// Per token t: latent = RMSNorm(katmp[:R]) * w (bit-exact with src/ops.c:76-83 up to the
// summation order of the double sum), stored fp32 and as hi/lo bf16; rotated k_rope
// (src/mla_prefill_streaming.c:131-138) stored fp32 [S, DR].
struct KvaEpiArgs {
    const float *y;
    const uint16_t *norm;
    const float2 *cs;
    float *latf;
    uint16_t *lath, *latl;
    float *krope;
    int *lat_flag;
    int ldy, koff, R, DR;
    float eps;
};

__global__ __launch_bounds__(256) void k_kva_epi(KvaEpiArgs a) {
    __shared__ double redd[256];
    const int t = blockIdx.x, tid = threadIdx.x, R = a.R, half = a.DR / 2;
    const float *kat = a.y + (size_t)t * a.ldy + a.koff;
    double ss = 0.0;
    for (int r = tid; r < R; r += 256) {
        const double v = (double)kat[r];
        ss += v * v;
    }
    redd[tid] = ss;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) redd[tid] += redd[tid + o];
        __syncthreads();
    }
    const float mean_sq = (float)(redd[0] / (double)R);
    const float inv = 1.0f / sqrtf(mean_sq + a.eps);
    int any = 0;
    for (int r = tid; r < R; r += 256) {
        const float v = kat[r] * inv;
        const float y = v * bf16_to_f32(a.norm[r]);
        a.latf[(size_t)t * R + r] = y;
        if (a.lath) {
            uint16_t h, l;
            split_bf16(y, h, l);
            a.lath[(size_t)t * R + r] = h;
            a.latl[(size_t)t * R + r] = l;
            any |= (l & 0x7fff) != 0;
        }
    }
    for (int i = tid; i < half; i += 256) {
        const float2 cs = a.cs[(size_t)t * half + i];
        const float ev = kat[R + 2 * i], od = kat[R + 2 * i + 1];
        const float ec = ev * cs.x, os = od * cs.y, oc = od * cs.x, es = ev * cs.y;
        a.krope[(size_t)t * a.DR + i] = ec - os;
        a.krope[(size_t)t * a.DR + half + i] = oc + es;
    }
    if (a.lat_flag && __syncthreads_or(any) && tid == 0) atomicOr(a.lat_flag, 1);
}

// Per (token t, head h): Q = [q_nope | RoPE(q_rope, t)] as hi/lo bf16 [NH, Sp, QD];
// K = [kv[t, h, :DN] | krope[t]] bf16 [NH, Sp, QD]; V^T bf16 [NH, DV, Sp].
struct PackArgs {
    const float *y, *kv, *krope;
    const float2 *cs;
    uint16_t *qh, *ql, *kb, *vt;
    int S, Sp, NH, DN, DR, DV, ldy;
};

__global__ __launch_bounds__(256) void k_pack(PackArgs a) {
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int QD = a.DN + a.DR, half = a.DR / 2;
    if (t >= a.S) {  // padding rows of the last tile: zero, so masked keys contribute 0 * 0
        const size_t qo = ((size_t)h * a.Sp + t) * QD;
        for (int k = tid; k < QD; k += 256) {
            a.qh[qo + k] = 0;
            a.ql[qo + k] = 0;
            a.kb[qo + k] = 0;
        }
        for (int d = tid; d < a.DV; d += 256) a.vt[((size_t)h * a.DV + d) * a.Sp + t] = 0;
        return;
    }
    const float *q = a.y + (size_t)t * a.ldy + (size_t)h * QD;
    const float *kv = a.kv + (size_t)t * a.NH * (a.DN + a.DV) + (size_t)h * (a.DN + a.DV);
    const size_t qo = ((size_t)h * a.Sp + t) * QD;
    for (int k = tid; k < QD; k += 256) {
        float qv;
        if (k < a.DN) {
            qv = q[k];
        } else {
            const int i = (k - a.DN) % half;
            const float2 cs = a.cs[(size_t)t * half + i];
            const float ev = q[a.DN + 2 * i], od = q[a.DN + 2 * i + 1];
            qv = (k - a.DN) < half ? ev * cs.x - od * cs.y : od * cs.x + ev * cs.y;
        }
        uint16_t hh, ll;
        split_bf16(qv, hh, ll);
        a.qh[qo + k] = hh;
        a.ql[qo + k] = ll;
        const float kvv = k < a.DN ? kv[k] : a.krope[(size_t)t * a.DR + (k - a.DN)];
        a.kb[qo + k] = f32_to_bf16_rne(kvv);
    }
    for (int d = tid; d < a.DV; d += 256)
        a.vt[((size_t)h * a.DV + d) * a.Sp + t] = f32_to_bf16_rne(kv[a.DN + d]);
}

// ================================================================ flash attention ======

// Causal attention for one head and 64 queries (4 waves x 16). QD = 192, DV = 128 here.
// S = Q K^T: M = 16 queries, N = 16 keys, K = 192 (6 x 32), Q as hi/lo bf16 (A), K bf16 (B).
// P = softmax rows (online), written per wave to LDS and re-read as the A operand (hi/lo).
// O += P V: N = 16 of the 128 value columns (8 tiles), K = 32 keys, V^T rows from LDS.
// Output rows normalised by l and written as hi/lo bf16 for the o_proj GEMM.
constexpr int kFQ = 64, kFK = 64;
constexpr int kFKs = 200;  // LDS K row: 192 + 8 bf16
constexpr int kFVs = 72;   // LDS V^T row: 64 + 8 bf16
constexpr int kFPs = 68;   // LDS P row: 64 + 4 fp32

struct FlashArgs {
    const uint16_t *qh, *ql, *kb, *vt;
    uint16_t *oh, *ol;  // [S, HO] hi/lo
    int S, Sp, NH, ldo;
    float smscale;
};

__global__ __launch_bounds__(256) void k_flash_prefill(FlashArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sk[kFK * kFKs];
    __shared__ __attribute__((aligned(16))) uint16_t sv[128 * kFVs];
    __shared__ __attribute__((aligned(16))) float sp[4][16 * kFPs];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, n = l & 15, g = l >> 4;
    const int nqt = (a.S + kFQ - 1) / kFQ;
    const int qt = nqt - 1 - (int)blockIdx.x;  // longest tiles first
    const int h = blockIdx.y;
    const int q0 = qt * kFQ;
    const size_t hq = (size_t)h * a.Sp;
    // Q operands: row q0 + 16w + n, dims kb*32 + 8g
    v8bf qa[6], qb[6];
    {
        const int qrow = q0 + 16 * w + n;
        const uint16_t *ph = a.qh + (hq + qrow) * 192;
        const uint16_t *pl = a.ql + (hq + qrow) * 192;
#pragma unroll
        for (int kb = 0; kb < 6; ++kb) {
            qa[kb] = *(const v8bf *)(ph + 32 * kb + 8 * g);
            qb[kb] = *(const v8bf *)(pl + 32 * kb + 8 * g);
        }
    }
    float m_run[4], l_run[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.f;
    }
    v4f acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
    const float sl2 = a.smscale * 1.4426950408889634f;  // exp(x) = exp2(x * log2 e)

    for (int kt = 0; kt <= qt; ++kt) {
        const int k0 = kt * kFK;
        __syncthreads();
        // K tile: 64 rows x 192 bf16 = 1536 x 16 B; V^T tile: 128 rows x 64 bf16 = 1024 x 16 B
        for (int p = tid; p < 64 * 24; p += 256) {
            const int row = p / 24, c8 = (p % 24) * 8;
            *(v4i *)(sk + row * kFKs + c8) = *(const v4i *)(a.kb + (hq + k0 + row) * 192 + c8);
        }
        for (int p = tid; p < 128 * 8; p += 256) {
            const int row = p >> 3, c8 = (p & 7) * 8;
            *(v4i *)(sv + row * kFVs + c8) = *(const v4i *)(a.vt + ((size_t)h * 128 + row) * a.Sp + k0 + c8);
        }
        __syncthreads();
        v4f s[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            s[nt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 6; ++kb) {
                const v8bf bk = *(const v8bf *)(sk + (16 * nt + n) * kFKs + 32 * kb + 8 * g);
                s[nt] = mfma_bf16(qa[kb], bk, s[nt]);
                s[nt] = mfma_bf16(qb[kb], bk, s[nt]);
            }
        }
        // D layout: query q0 + 16w + 4g + i, key k0 + 16nt + n
        float mx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qi = q0 + 16 * w + 4 * g + i;
            float m = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const int kj = k0 + 16 * nt + n;
                float v = s[nt][i] * sl2;
                if (kj > qi || kj >= a.S) v = -INFINITY;
                s[nt][i] = v;
                m = fmaxf(m, v);
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
            mx[i] = m;
        }
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float mnew = fmaxf(m_run[i], mx[i]);
            alpha[i] = exp2f(m_run[i] - mnew);
            m_run[i] = mnew;
            float ps = 0.f;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const float p = exp2f(s[nt][i] - mnew);
                ps += p;
                sp[w][(4 * g + i) * kFPs + 16 * nt + n] = p;
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) ps += __shfl_xor(ps, o);
            l_run[i] = fmaf(l_run[i], alpha[i], ps);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] *= alpha[i];
        __syncthreads();  // P rows of this wave are visible in LDS
        // P as A operand: query n, keys kb2*32 + 8g .. +7
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) {
            const float *pr = &sp[w][n * kFPs + 32 * kb2 + 8 * g];
            const v4f p0 = *(const v4f *)pr, p1 = *(const v4f *)(pr + 4);
            v8bf ph, pl;
            split8(p0, p1, ph, pl);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const v8bf bv = *(const v8bf *)(sv + (16 * t + n) * kFVs + 32 * kb2 + 8 * g);
                acc[t] = mfma_bf16(ph, bv, acc[t]);
                acc[t] = mfma_bf16(pl, bv, acc[t]);
            }
        }
    }
    float inv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) inv[i] = 1.0f / l_run[i];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qi = q0 + 16 * w + 4 * g + i;
            if (qi >= a.S) continue;
            const float v = acc[t][i] * inv[i];
            uint16_t hh, ll;
            split_bf16(v, hh, ll);
            const size_t o = (size_t)qi * a.ldo + (size_t)h * 128 + 16 * t + n;
            a.oh[o] = hh;
            a.ol[o] = ll;
        }
}

// ================================================================ generic route ========

// Per token: RMSNorm latent, rotated k_rope, and Q rows [S, NH, QD] fp32 (any dims).
struct GenEpiArgs {
    const float *y;
    const uint16_t *norm;
    const float2 *cs;
    float *latf, *krope, *qf;
    int ldy, NH, DN, DR, R, QO;
    float eps;
};

__global__ __launch_bounds__(256) void k_gen_epi(GenEpiArgs a) {
    const int t = blockIdx.x, tid = threadIdx.x, half = a.DR / 2, QD = a.DN + a.DR;
    const float *row = a.y + (size_t)t * a.ldy;
    for (int i = tid; i < a.NH * QD; i += 256) {
        const int h = i / QD, k = i % QD;
        const float *q = row + (size_t)h * QD;
        float v;
        if (k < a.DN) {
            v = q[k];
        } else {
            const int j = (k - a.DN) % half;
            const float2 cs = a.cs[(size_t)t * half + j];
            const float ev = q[a.DN + 2 * j], od = q[a.DN + 2 * j + 1];
            const float ec = ev * cs.x, os = od * cs.y, oc = od * cs.x, es = ev * cs.y;
            v = (k - a.DN) < half ? ec - os : oc + es;
        }
        a.qf[(size_t)t * a.NH * QD + i] = v;
    }
    (void)a.QO;
}

// Causal attention, one block per (query t, head h), any dims; scores in global scratch.
struct GenAttnArgs {
    const float *qf, *kv, *krope;
    float *heads, *scr;
    int S, NH, DN, DR, DV;
    float smscale;
};

__global__ __launch_bounds__(256) void k_gen_attn(GenAttnArgs a) {
    __shared__ float red[256];
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int QD = a.DN + a.DR, KH = a.DN + a.DV, L = t + 1;
    const float *q = a.qf + ((size_t)t * a.NH + h) * QD;
    float *sc = a.scr + ((size_t)t * a.NH + h) * a.S;
    for (int j = tid; j < L; j += 256) {
        const float *kj = a.kv + (size_t)j * a.NH * KH + (size_t)h * KH;
        const float *rj = a.krope + (size_t)j * a.DR;
        float acc = 0.f;
        for (int k = 0; k < a.DN; ++k) acc = fmaf(q[k], kj[k], acc);
        for (int k = 0; k < a.DR; ++k) acc = fmaf(q[a.DN + k], rj[k], acc);
        sc[j] = acc * a.smscale;
    }
    __syncthreads();
    float m = -INFINITY;
    for (int j = tid; j < L; j += 256) m = fmaxf(m, sc[j]);
    red[tid] = m;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    m = red[0];
    __syncthreads();
    float sum = 0.f;
    for (int j = tid; j < L; j += 256) {
        const float e = __expf(sc[j] - m);
        sc[j] = e;
        sum += e;
    }
    red[tid] = sum;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] += red[tid + o];
        __syncthreads();
    }
    const float inv = 1.0f / red[0];
    for (int d = tid; d < a.DV; d += 256) {
        float acc = 0.f;
        for (int j = 0; j < L; ++j) acc = fmaf(sc[j], a.kv[(size_t)j * a.NH * KH + (size_t)h * KH + a.DN + d], acc);
        a.heads[(size_t)t * a.NH * a.DV + (size_t)h * a.DV + d] = acc * inv;
    }
}

// ================================================================ driver ===============

hipError_t launch_gemv(hipStream_t st, float *Y, int ldy, const float *X, int ldx, int B,
                       const uint16_t *W0, int out0, const uint16_t *W1, int out1, int in,
                       bool accumulate);

bool prefill_mfma_shape(const Dims &d) {
    return d.H % 32 == 0 && d.R % 32 == 0 && d.QD == 192 && d.DV == 128 && d.HO % 32 == 0 &&
           d.DN % 8 == 0;
}

size_t prefill_bytes(const Dims &d, int S) {
    const size_t Sp = (size_t)(S + 63) / 64 * 64;
    size_t b = 0;
    auto add = [&](size_t n) { b += (n + 255) / 256 * 256 + 256; };
    if (prefill_mfma_shape(d)) {
        add(4 * 8);                              // flags
        add(2 * (size_t)S * d.H * 2);            // x hi/lo
        add(4 * (size_t)S * (d.QO + d.KVO));     // y
        add(4 * (size_t)S * d.R);                // latf
        add(2 * 2 * (size_t)S * d.R);            // lat hi/lo
        add(4 * (size_t)S * d.DR);               // krope
        add(4 * (size_t)S * d.KVB);              // kv
        add(2 * 2 * (size_t)d.NH * Sp * d.QD);   // q hi/lo
        add(2 * (size_t)d.NH * Sp * d.QD);       // k
        add(2 * (size_t)d.NH * d.DV * Sp);       // v^T
        add(2 * 2 * (size_t)S * d.HO);           // heads hi/lo
    } else {
        add(4 * (size_t)S * (d.QO + d.KVO));
        add(4 * (size_t)S * d.R);
        add(4 * (size_t)S * d.DR);
        add(4 * (size_t)S * d.NH * d.QD);
        add(4 * (size_t)S * d.KVB);
        add(4 * (size_t)S * d.HO);
        add(4 * (size_t)S * d.NH * S);
    }
    return b;
}

hipError_t launch_prefill_all(hipStream_t st, const Dims &d, int S, float eps, const float *x,
                              float *out, const uint16_t *wq, const uint16_t *wkva,
                              const uint16_t *wnorm, const uint16_t *wkvb, const uint16_t *wo,
                              const float2 *cs, void *ws) {
    const int Sp = (S + 63) / 64 * 64;
    char *base = (char *)ws;
    size_t off = 0;
    auto take = [&](size_t n) {
        off = (off + 255) / 256 * 256;
        void *p = base + off;
        off += n + 256;
        return p;
    };
    const float smscale = 1.0f / sqrtf((float)d.QD);
    const int ldy = d.QO + d.KVO;
    hipError_t e;
    if (prefill_mfma_shape(d)) {
        int *flags = (int *)take(4 * 8);
        uint16_t *xh = (uint16_t *)take(2 * (size_t)S * d.H);
        uint16_t *xl = (uint16_t *)take(2 * (size_t)S * d.H);
        float *y = (float *)take(4 * (size_t)S * ldy);
        float *latf = (float *)take(4 * (size_t)S * d.R);
        uint16_t *lath = (uint16_t *)take(2 * (size_t)S * d.R);
        uint16_t *latl = (uint16_t *)take(2 * (size_t)S * d.R);
        float *krope = (float *)take(4 * (size_t)S * d.DR);
        float *kv = (float *)take(4 * (size_t)S * d.KVB);
        uint16_t *qh = (uint16_t *)take(2 * (size_t)d.NH * Sp * d.QD);
        uint16_t *ql = (uint16_t *)take(2 * (size_t)d.NH * Sp * d.QD);
        uint16_t *kb = (uint16_t *)take(2 * (size_t)d.NH * Sp * d.QD);
        uint16_t *vt = (uint16_t *)take(2 * (size_t)d.NH * d.DV * Sp);
        uint16_t *oh = (uint16_t *)take(2 * (size_t)S * d.HO);
        uint16_t *ol = (uint16_t *)take(2 * (size_t)S * d.HO);
        hipLaunchKernelGGL(k_zero_int, dim3(1), dim3(64), 0, st, flags, 8);
        hipLaunchKernelGGL(k_split, dim3(1024), dim3(256), 0, st, x, d.H, xh, xl, d.H, S, d.H, flags + 0);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = gemm(st, xh, xl, flags + 0, d.H, wq, d.H, y, ldy, S, d.QO, d.H)) != hipSuccess) return e;
        if ((e = gemm(st, xh, xl, flags + 0, d.H, wkva, d.H, y + d.QO, ldy, S, d.KVO, d.H)) != hipSuccess)
            return e;
        KvaEpiArgs ea{y, wnorm, cs, latf, lath, latl, krope, flags + 1, ldy, d.QO, d.R, d.DR, eps};
        hipLaunchKernelGGL(k_kva_epi, dim3(S), dim3(256), 0, st, ea);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = gemm(st, lath, latl, flags + 1, d.R, wkvb, d.R, kv, d.KVB, S, d.KVB, d.R)) != hipSuccess)
            return e;
        PackArgs pa{y, kv, krope, cs, qh, ql, kb, vt, S, Sp, d.NH, d.DN, d.DR, d.DV, ldy};
        hipLaunchKernelGGL(k_pack, dim3(Sp, d.NH), dim3(256), 0, st, pa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        FlashArgs fa{qh, ql, kb, vt, oh, ol, S, Sp, d.NH, d.HO, smscale};
        hipLaunchKernelGGL(k_flash_prefill, dim3(Sp / 64, d.NH), dim3(256), 0, st, fa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // attention outputs are never bf16-exact: the lo pass always runs (no flag)
        if ((e = gemm(st, oh, ol, nullptr, d.HO, wo, d.HO, out, d.H, S, d.H, d.HO)) != hipSuccess) return e;
        return hipSuccess;
    }
    float *y = (float *)take(4 * (size_t)S * ldy);
    float *latf = (float *)take(4 * (size_t)S * d.R);
    float *krope = (float *)take(4 * (size_t)S * d.DR);
    float *qf = (float *)take(4 * (size_t)S * d.NH * d.QD);
    float *kv = (float *)take(4 * (size_t)S * d.KVB);
    float *heads = (float *)take(4 * (size_t)S * d.HO);
    float *scr = (float *)take(4 * (size_t)S * d.NH * S);
    if ((e = launch_gemv(st, y, ldy, x, d.H, S, wq, d.QO, wkva, d.KVO, d.H, false)) != hipSuccess) return e;
    KvaEpiArgs ea{y, wnorm, cs, latf, nullptr, nullptr, krope, nullptr, ldy, d.QO, d.R, d.DR, eps};
    hipLaunchKernelGGL(k_kva_epi, dim3(S), dim3(256), 0, st, ea);
    GenEpiArgs ga{y, wnorm, cs, latf, krope, qf, ldy, d.NH, d.DN, d.DR, d.R, d.QO, eps};
    hipLaunchKernelGGL(k_gen_epi, dim3(S), dim3(256), 0, st, ga);
    if ((e = launch_gemv(st, kv, d.KVB, latf, d.R, S, wkvb, d.KVB, nullptr, 0, d.R, false)) != hipSuccess)
        return e;
    GenAttnArgs aa{qf, kv, krope, heads, scr, S, d.NH, d.DN, d.DR, d.DV, smscale};
    hipLaunchKernelGGL(k_gen_attn, dim3(S, d.NH), dim3(256), 0, st, aa);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return launch_gemv(st, out, d.H, heads, d.HO, S, wo, d.H, nullptr, 0, d.HO, false);
}

}  // namespace kvl
