// HIP kernels of the causal MLA prefill (src/mla_prefill_streaming.c:78-206 of the
// reference: non-absorbed attention, K/V expanded through kv_b for every token).
//
// MFMA route (H, R and NH * DV multiples of 64, QD = 192, DV = 128, DN multiple of 8):
//   split     x (fp32) -> bf16 hi + lo operands; a flag records whether any lo is non-zero
//   gemm      [q | kv_a] = x . W^T           (bf16 MFMA, fp32 accumulate, lo pass skipped
//                                             when the operand is exactly bf16); epilogue:
//                                             Q = [q_nope | RoPE(q_rope)] as hi/lo fp16
//   kva_pack  RMSNorm -> latent (hi/lo bf16), RoPE(k_rope) -> rope part of K (fp16 hi + K8)
//   gemm      kv = latent . kv_b^T           epilogue: k_nope -> K (fp16 hi + K8), V^T (fp16)
//   flash     causal attention per (128-query tile, head), online softmax; scores Kh Qh in
//             fp16 plus the Kh Ql + Kl Qh correction from bf8 operands (K8: bf8 of the hi
//             parts and of the lo parts x 2^11)
//   gemm      out = heads . o_proj^T          (fp16 heads and fp16 copy of o_proj, one pass)
// Generic route (any shape): the same stages with VALU kernels.
//
// Range of the 16-bit operands. V (and so the attention output) and the fp16 o_proj copy carry
// power-of-two scales chosen by the host from bounds it knows (|V| <= sqrt(R) max|norm weight|
// max ||kv_b row||_2; max|o_proj|), undone exactly by the o_proj epilogue. Q and K depend on x
// and are not scaled; the flash kernel checks every query row instead: a row whose reference
// max logit exceeds kFLogitMax (beyond it the bf8 score correction's error grows past the 2e-3
// budget) or whose output is not finite raises a per-call flag (and a sticky flag for callers
// that read it later). The o_proj epilogue then writes NaN, and the host-buffer entry points
// run the call again on the generic route.
#include "mla_device.h"
#include "mla_internal.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace kvl {

// ================================================================ split ================

// src[r, c] (fp32, ld_src) -> hi/lo bf16 [rows, cols] (ld_dst); flag |= any lo != 0.
// Each thread converts 8 consecutive values (cols % 8 == 0, 16-byte aligned rows).
__global__ __launch_bounds__(256) void k_split(const float *src, int ld_src, uint16_t *hi,
                                               uint16_t *lo, int ld_dst, int rows, int cols,
                                               int *flag) {
    const int c8 = cols / 8;
    int any = 0;
    // flag[1]: the range flag of this call (raised by the flash kernel, read by the o_proj
    // epilogue), cleared here, in the call's first kernel
    if (flag && blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(flag + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    // rows over blocks, 8-column groups over threads (no index division in the loop)
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *s = src + (size_t)r * ld_src;
        uint16_t *hr = hi + (size_t)r * ld_dst, *lr = lo + (size_t)r * ld_dst;
        for (int c = 8 * threadIdx.x; c < 8 * c8; c += 8 * 256) {
            const v4f x0 = *(const v4f *)(s + c), x1 = *(const v4f *)(s + c + 4);
            v8bf h, l;
            split8(x0, x1, h, l);
            *(v8bf *)(hr + c) = h;
            *(v8bf *)(lr + c) = l;
            const v4i lv = __builtin_bit_cast(v4i, l);
            any |= ((lv.x | lv.y | lv.z | lv.w) & 0x7fff7fff) != 0;
        }
    }
    // Blocks with a non-zero lo word store 1. Every writer stores the same value and the reader
    // is a later kernel, so a workgroup-scope store (cached in the XCD's L2, written back at
    // the kernel's end) suffices; device-coherent stores or atomics to one address from every
    // block serialise at memory (measured 13-65 us for 2048 blocks). The flag is only raised
    // here; k_kva_pack clears it after the q GEMM has read it.
    if (flag && __syncthreads_or(any) && threadIdx.x == 0)
        __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ================================================================ GEMM =================

// C[m, n] = sum_k (Ah + Al)[m, k] * B[n, k]: row-major bf16 operands, fp32 output. The
// columns of C may come from two weight matrices (B0 for n < N0, B1 for the N1 after it),
// so the q and kv_a projections of the same tokens run as one launch.
//
// Block tile 256 x BN (BN = 256 or 128), eight math waves (2 per SIMD) in a WM x WN grid, each
// owning a (256 / WM) x (BN / WN) quadrant of v_mfma_f32_16x16x32 tiles. Large tiles keep
// the L2 traffic at 24-32 bytes per clock per CU at the MFMA rate. The lo operand, when it
// is given and needed, is a second pass over k: the k loop runs over [Ah | Al] against
// [B | B], so each stage is one A and one B tile with a k step of 64, and all stages have
// the same shape. They stream into an LDS ring of 3 stages (2 where 3 do not fit) by
// global_load_lds_dwordx4 DMA, issued by four more waves that do nothing else: a DMA
// instruction holds its wave until the memory system accepts it (about a quarter of a math
// wave's time when the math waves issued their own), so the math waves only compute and meet
// the DMA waves at one barrier per stage (the DMA waves wait for stage kt's data before it).
// 128-byte rows with slot s at s ^ (r & 7) spread the 8 rows one ds_read_b128 phase touches
// over distinct banks. Each wave reads all its fragments of a 32-deep k-sub before its MFMAs.
// The lo pass runs when Al is given and either no flag is given or *lo_flag != 0 (the flag
// is raised by the producer of Al when some lo word is non-zero). Requires K % 64 == 0, lda
// and ldb multiples of 8.
constexpr int kGBm = 256;
constexpr int kGemmMath = 8, kGemmDma = 4;  // waves of a GEMM block

template <int BN>
struct GemmShape {
    static constexpr int BK = 64, RowB = BK * 2, Spr = BK / 8;  // 16-byte slots per row
    static constexpr int WM = BN == 256 ? 2 : 4, WN = 8 / WM;
    static constexpr int TM = kGBm / WM / 16, TN = BN / WN / 16;  // 16x16 tiles per wave
    static constexpr int ATile = kGBm * RowB, BTile = BN * RowB;
    static constexpr int Stage = ATile + BTile;
    static constexpr int Stages = (160 * 1024) / Stage >= 3 ? 3 : 2;  // ring depth that fits
    static constexpr int Smem = Stages * Stage;
    __device__ static int swz(int row) { return row & 7; }
};

struct GemmArgs {
    const uint16_t *Ah, *Al, *B0, *B1;
    float *C;
    const int *lo_flag;
    int M, N0, N1, K, lda, ldb, ldc;
};

// Epilogues. kEpiPlain: C fp32. kEpiQ (q | kv_a projection): the N0 = NH * QD q columns go
// to Q [NH, Sp, QD] as hi/lo fp16 with the rope half rotated (src/mla_prefill_streaming.c:
// 139-147: pairs (2i, 2i+1) -> i and DR/2 + i), the kv_a columns to C (ldc = N1). kEpiKV
// (kv_b projection): k_nope -> K hi [NH, Sp, QD] fp16 and K8 [NH, Sp, 384 bytes] (bf8 of the
// hi parts and of the lo parts x 2^11, k8_hi_byte order), values -> V^T [NH, DV, Sp] fp16 with
// the keys of each 32-key group in vt_perm order.
enum { kEpiPlain = 0, kEpiQ = 1, kEpiKV = 2 };
struct GemmEpi {
    _Float16 *qh, *kh;
    uint8_t *ql8;  // bf8(Q lo x 2^11), the flash kernel's correction operand (kEpiQ)
    uint8_t *k8;
    _Float16 *vt;
    const float2 *cs;
    int Sp, DN, DR, DV;
    float vscale = 1.0f;             // kEpiKV: V^T = vscale * v (a power of two)
    float alpha = 1.0f;              // kEpiPlain: C = alpha * acc (a power of two)
    const int *nan_flag = nullptr;   // kEpiPlain: C = NaN when *nan_flag != 0
};

// Position of key k (0..31 within its 32-key group) in the permuted V^T rows: the 8 keys
// lane group g of the flash kernel holds for one PV chunk are 4g .. 4g+3 and 16+4g .. 16+4g+3.
__host__ __device__ __forceinline__ int vt_perm(int k) { return 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3); }

// F16: the 16-bit operands are fp16 (v_mfma_f32_16x16x32_f16) instead of bf16.
template <bool F16>
__device__ __forceinline__ v4f mfma16(const v8bf &a, const v8bf &b, const v4f &c) {
    if constexpr (F16) return mfma_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c);
    else return mfma_bf16(a, b, c);
}

// s_waitcnt vmcnt(PER * min(later, MAXL)) for a wave-uniform count of later stages in flight.
template <int PER, int MAXL>
__device__ __forceinline__ void wait_stages(int later) {
    if constexpr (MAXL == 0) {
        wait_vmcnt<0>();
    } else {
        if (later >= MAXL) wait_vmcnt<PER * MAXL>();
        else wait_stages<PER, MAXL - 1>(later);
    }
}

template <int BN, int EPI, bool F16>
__global__ __launch_bounds__(64 * (kGemmMath + kGemmDma)) void k_gemm16(GemmArgs a, GemmEpi e) {
    using Sh = GemmShape<BN>;
    constexpr int BK = Sh::BK, RowB = Sh::RowB, Spr = Sh::Spr;
    constexpr int TM = Sh::TM, TN = Sh::TN;
    __shared__ __attribute__((aligned(16))) uint8_t smem[Sh::Smem];
    const uint32_t sbase = lds_addr(smem);
    const int tid = threadIdx.x, l = tid & 63, n = l & 15, g = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w / Sh::WN, wn = w % Sh::WN;
    const int M = a.M, N0 = a.N0, N1 = a.N1, K = a.K, lda = a.lda, ldb = a.ldb;
    const int tn0 = (N0 + BN - 1) / BN, tn = tn0 + (N1 + BN - 1) / BN;
    const int tm = (M + kGBm - 1) / kGBm, ntiles = tm * tn;
    // Tiles in row-major order; with ntiles % 8 == 0, XCD b % 8 takes a contiguous eighth
    // of them (blocks of one XCD share A rows in its L2).
    int tile = blockIdx.x;
    if (ntiles % 8 == 0) tile = (blockIdx.x & 7) * (ntiles / 8) + (blockIdx.x >> 3);
    const int mt = tile / tn, nt = tile % tn;
    const bool seg1 = nt >= tn0;
    const uint16_t *B = seg1 ? a.B1 : a.B0;
    const int Nseg = seg1 ? N1 : N0;
    const int nb0 = seg1 ? (nt - tn0) * BN : nt * BN;  // first row of B in this tile
    const int c0 = seg1 ? N0 + nb0 : nb0;              // first column of C
    const int m0 = mt * kGBm;
    const bool use_lo = a.Al && (!a.lo_flag || *a.lo_flag);

    const int nk = K / BK, nkt = use_lo ? 2 * nk : nk;  // k steps of the hi pass, of all passes
    constexpr int NS = Sh::Stages;
    if (w >= kGemmMath) {
        // DMA wave dw: instruction i fills slot (4i + dw) * 64 + l of a tile: row p / Spr,
        // physical slot p % Spr holding logical slot (p % Spr) ^ swz(row). Rows past the end of
        // A or B are clamped to the last row (their results are never stored).
        const int dw = w - kGemmMath;
        constexpr int NA = Sh::ATile / (kGemmDma * 1024), NB = Sh::BTile / (kGemmDma * 1024);
        uint32_t aoff[NA], boff[NB];
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int p = (kGemmDma * i + dw) * 64 + l, row = p / Spr, s = (p % Spr) ^ Sh::swz(row);
            aoff[i] = (uint32_t)(min(m0 + row, M - 1) - m0) * lda * 2 + 16 * s;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int p = (kGemmDma * i + dw) * 64 + l, row = p / Spr, s = (p % Spr) ^ Sh::swz(row);
            boff[i] = (uint32_t)(min(nb0 + row, Nseg - 1) - nb0) * ldb * 2 + 16 * s;
        }
        const uint8_t *gah = (const uint8_t *)(a.Ah + (size_t)m0 * lda);
        const uint8_t *gal = use_lo ? (const uint8_t *)(a.Al + (size_t)m0 * lda) : gah;
        const uint8_t *gb = (const uint8_t *)(B + (size_t)nb0 * ldb);
        auto issue = [&](int kt, int stage) __attribute__((always_inline)) {
            const uint32_t dst = sbase + stage * Sh::Stage + (uint32_t)dw * 1024;
            const bool lo = kt >= nk;
            const uint8_t *ga = lo ? gal : gah;
            const size_t ko = (size_t)(lo ? kt - nk : kt) * BK * 2;
#pragma unroll
            for (int i = 0; i < NA; ++i) dma_b128_s(ga + ko, aoff[i], dst + i * (kGemmDma * 1024));
#pragma unroll
            for (int i = 0; i < NB; ++i) dma_b128_s(gb + ko, boff[i], dst + Sh::ATile + i * (kGemmDma * 1024));
        };
#pragma unroll
        for (int q = 0; q < NS - 1; ++q)
            if (q < nkt) issue(q, q);
        for (int kt = 0; kt < nkt; ++kt) {
            // stage kt has landed when at most min(NS - 2, nkt - 1 - kt) later stages are in flight
            wait_stages<NA + NB, NS - 2>(min(NS - 2, nkt - 1 - kt));
            lds_barrier();  // stage kt is in LDS; every math wave is done with stage kt - 1
            if (kt + NS - 1 < nkt) issue(kt + NS - 1, (kt + NS - 1) % NS);
        }
        lds_barrier();  // the math waves' epilogue barrier
        return;
    }
    // fragment rows 16 * tile + n (n & 7 = row & 7), logical slot 4 ks + g of k-sub ks
    int frd[BK / 32];
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) frd[ks] = n * RowB + 16 * ((4 * ks + g) ^ Sh::swz(n));

    v4f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int kt = 0; kt < nkt; ++kt) {
        lds_barrier();  // stage kt has landed (the DMA waves waited for it)
        const uint8_t *st = smem + (kt % NS) * Sh::Stage;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const uint8_t *sa = st + wm * (TM * 16) * RowB + frd[ks];
            const uint8_t *sb = st + Sh::ATile + wn * (TN * 16) * RowB + frd[ks];
            v8bf bo[TN], ao[TM];
#pragma unroll
            for (int j = 0; j < TN; ++j) bo[j] = *(const v8bf *)(sb + j * 16 * RowB);
#pragma unroll
            for (int i = 0; i < TM; ++i) ao[i] = *(const v8bf *)(sa + i * 16 * RowB);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma16<F16>(ao[i], bo[j], acc[i][j]);
        }
    }
    // Epilogue. D layout: lane (g, n) of tile (i, j) holds rows 4g + r, column n. Row-major
    // outputs go through a per-wave LDS buffer (16 rows x 64 columns per tile row i): lane l
    // then takes columns 4 (l % 16) .. + 3 of rows l / 16 + 4 q, q = 0..3, so the 16 lanes of a
    // row write its 64 columns as one contiguous run (scattered 16-byte pieces per lane cost
    // ~10 us more per launch at these sizes), and the rope pairs (2p, 2p+1) sit in one lane.
    // The V^T part of kEpiKV wants 4 consecutive tokens per lane, which the D layout gives.
    const int QD = e.DN + e.DR, KH = e.DN + e.DV, half = e.DR / 2;
    static_assert(TN == 4, "the staged epilogue assumes 64 columns per wave");
    lds_barrier();  // every wave is done with the ring
    float *ep = (float *)smem + w * (16 * 68);
    const int cw = wn * 64;                      // wave's first column within the tile
    const bool vt_wave = EPI == kEpiKV && ((nb0 + cw) % KH) >= e.DN;
    const int rr = l >> 4, cc = (l & 15) * 4;    // staged row (+ 4 q) / first column of this lane
    const int nl0 = nb0 + cw + cc;               // segment column of v[0]
    float alpha = e.alpha;
    if (EPI == kEpiPlain && e.nan_flag && __hip_atomic_load(e.nan_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        alpha = __builtin_nanf("");
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int rbase = m0 + wm * TM * 16 + 16 * i;
        if (vt_wave) {
            const int row0 = rbase + 4 * g;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int nl = nb0 + cw + 16 * j + n;
                if (nl >= Nseg) continue;
                const int h = nl / KH, d = nl % KH - e.DN;
                const v4h hv = {(_Float16)(acc[i][j][0] * e.vscale), (_Float16)(acc[i][j][1] * e.vscale),
                                (_Float16)(acc[i][j][2] * e.vscale), (_Float16)(acc[i][j][3] * e.vscale)};
                const size_t o = ((size_t)h * e.DV + d) * e.Sp + (row0 & ~31) + vt_perm(row0 & 31);
                if (row0 + 3 < M) {
                    *(v4h *)(e.vt + o) = hv;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (row0 + r < M) e.vt[o + r] = hv[r];
                }
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) ep[(4 * g + r) * 68 + 16 * j + n] = acc[i][j][r];
        v4f vq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) vq[q] = *(const v4f *)(ep + (rr + 4 * q) * 68 + cc);
        if (nl0 >= Nseg) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int t = rbase + rr + 4 * q;
            if (t >= M) continue;
            const float v[4] = {vq[q].x, vq[q].y, vq[q].z, vq[q].w};
            if (EPI == kEpiPlain || (EPI == kEpiQ && seg1)) {
                float *dst = EPI == kEpiPlain ? a.C + (size_t)t * a.ldc + c0 + cw + cc : a.C + (size_t)t * a.ldc + nl0;
                *(v4f *)dst = EPI == kEpiPlain ? vq[q] * alpha : vq[q];
            } else if (EPI == kEpiQ) {
                // Q (50 MB at 4096 tokens) is read once, by the flash kernel's workgroup of its
                // query tile: non-temporal stores keep it from evicting the K/V and weight
                // lines the next kernels reuse (q GEMM 78 -> 70 us, kv_b GEMM 44 -> 40 us)
                const int h = nl0 / QD, k0 = nl0 % QD;
                const size_t o = ((size_t)h * e.Sp + t) * QD;
                // Q hi as fp16 and Q lo only as the bf8 byte the flash kernel's correction takes
                // (bf8(lo x 2^11)): 37.5 instead of 50 MB written at 4096 tokens
                if (k0 < e.DN) {
                    v4h hi;
                    uint32_t l8 = 0;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        _Float16 hh, ll;
                        split_f16(v[u], hh, ll);
                        hi[u] = hh;
                        l8 |= bf8_lo_s11(ll) << (8 * u);
                    }
                    __builtin_nontemporal_store(hi, (v4h *)(e.qh + o + k0));
                    __builtin_nontemporal_store(l8, (uint32_t *)(e.ql8 + o + k0));
                } else {
                    // pairs (ev, od) = (v[2p], v[2p+1]) of rope index i2 + p
                    const int i2 = (k0 - e.DN) >> 1;
                    const float2 *cs = e.cs + (size_t)t * half + i2;
                    v2h h0, h1;
                    uint16_t l0 = 0, l1 = 0;
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const float2 c = cs[p];
                        const float ev = v[2 * p], od = v[2 * p + 1];
                        _Float16 hh, ll;
                        split_f16(ev * c.x - od * c.y, hh, ll);
                        h0[p] = hh;
                        l0 |= (uint16_t)(bf8_lo_s11(ll) << (8 * p));
                        split_f16(od * c.x + ev * c.y, hh, ll);
                        h1[p] = hh;
                        l1 |= (uint16_t)(bf8_lo_s11(ll) << (8 * p));
                    }
                    __builtin_nontemporal_store(h0, (v2h *)(e.qh + o + e.DN + i2));
                    __builtin_nontemporal_store(l0, (uint16_t *)(e.ql8 + o + e.DN + i2));
                    __builtin_nontemporal_store(h1, (v2h *)(e.qh + o + e.DN + half + i2));
                    __builtin_nontemporal_store(l1, (uint16_t *)(e.ql8 + o + e.DN + half + i2));
                }
            } else {  // kEpiKV, k_nope columns
                const int h = nl0 / KH, k0 = nl0 % KH;
                const size_t o = ((size_t)h * e.Sp + t) * QD + k0;
                v4h hi;
                uint32_t h8 = 0, l8 = 0;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    _Float16 hh, ll;
                    split_f16(v[u], hh, ll);
                    hi[u] = hh;
                    h8 |= f16_to_bf8(hh) << (8 * u);
                    l8 |= bf8_lo_s11(ll) << (8 * u);
                }
                *(v4h *)(e.kh + o) = hi;
                uint8_t *row = e.k8 + ((size_t)h * e.Sp + t) * 384 + k8_hi_byte(k0);
                *(uint32_t *)row = h8;
                *(uint32_t *)(row + kK8Lo) = l8;
            }
        }
    }
}

// C = A . [B0; B1]^T with N0 + N1 output columns (N1 = 0: a single weight matrix). One block
// per CU: the 256 x 256 tile is used unless 256 x 128 tiles (half the work each) need fewer
// than twice as many rounds over the 256 CUs.
template <int EPI, bool F16 = false>
static hipError_t gemm(hipStream_t st, const uint16_t *Ah, const uint16_t *Al, const int *flag,
                       int lda, const uint16_t *B0, int N0, const uint16_t *B1, int N1, int ldb,
                       float *C, int ldc, int M, int K, const GemmEpi &e) {
    GemmArgs a{Ah, Al, B0, B1 ? B1 : B0, C, flag, M, N0, N1, K, lda, ldb, ldc};
    const int tm = (M + kGBm - 1) / kGBm;
    const int t256 = tm * ((N0 + 255) / 256 + (N1 + 255) / 256);
    const int t128 = tm * ((N0 + 127) / 128 + (N1 + 127) / 128);
    const bool big = 2 * ((t256 + 255) / 256) <= (t128 + 255) / 256;
    if (K % 64) return hipErrorInvalidValue;
    constexpr int nt = 64 * (kGemmMath + kGemmDma);
    if (big) hipLaunchKernelGGL((k_gemm16<256, EPI, F16>), dim3(t256), dim3(nt), 0, st, a, e);
    else hipLaunchKernelGGL((k_gemm16<128, EPI, F16>), dim3(t128), dim3(nt), 0, st, a, e);
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

// MFMA route, one wave per token t: latent = RMSNorm(kv_a[t, :R]) * w (as k_kva_epi) as
// hi/lo bf16 [S, R] for the kv_b GEMM (whose lo pass always runs), and the rotated k_rope
// (src/mla_prefill_streaming.c:131-138) into the rope part of K for every head, as the fp16
// hi row and the K8 bytes (bf8 of hi and of lo x 2^11). Tokens S .. Sp-1 zero their Q, K, K8
// and V^T entries, so padding keys contribute 0 * 0 in the flash kernel.
struct KvaPackArgs {
    const float *y;  // [S, ldy] kv_a projection
    const uint16_t *norm;
    const float2 *cs;
    uint16_t *lath, *latl;
    _Float16 *qh;
    uint8_t *ql8;
    _Float16 *kh;
    uint8_t *k8;
    _Float16 *vt;
    size_t pstride;  // np partials of y, pstride floats apart, summed in order
    int np, S, Sp, NH, ldy, R, DN, DR, DV;
    float eps;
    int *x_flag;     // the x lo flag, cleared for the next prefill (its one reader has run)
};

__global__ __launch_bounds__(256) void k_kva_pack(KvaPackArgs a) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.x_flag) *a.x_flag = 0;
    if (t >= a.Sp) return;
    const int QD = a.DN + a.DR, half = a.DR / 2, R = a.R;
    if (t >= a.S) {
        const int tv = (t & ~31) | vt_perm(t & 31);
        for (int h = 0; h < a.NH; ++h) {
            const size_t qo = ((size_t)h * a.Sp + t) * QD;
            for (int k = l; k < QD; k += 64) {
                a.qh[qo + k] = 0;
                a.ql8[qo + k] = 0;
                a.kh[qo + k] = 0;
            }
            for (int k = l; k < 96; k += 64) ((uint32_t *)(a.k8 + ((size_t)h * a.Sp + t) * 384))[k] = 0;
            for (int d = l; d < a.DV; d += 64) a.vt[((size_t)h * a.DV + d) * a.Sp + tv] = 0;
        }
        return;
    }
    const float *kat = a.y + (size_t)t * a.ldy;
    if (R == 512 && a.DR == 64 && (a.DN & 63) == 0 && (a.ldy & 3) == 0 && (a.pstride & 3) == 0) {
        // lane l: latent columns 8l .. 8l+7 (16-byte loads and stores); the rotated RoPE key
        // goes through LDS so that each head's 128-byte fp16 hi row and its 128 K8 bytes (the
        // rope dims are k-block pair DN / 64: 4 hi slots, 4 lo slots) are written by 16 lanes of
        // 16 bytes, four heads per store instruction
        __shared__ __attribute__((aligned(16))) _Float16 rp[4][64];
        __shared__ __attribute__((aligned(16))) uint8_t k8p[4][8][16];  // [wave][part * 4 + g]
        const int w = threadIdx.x >> 6;
        float v[8];
        {
            v4f p0 = *(const v4f *)(kat + 8 * l), p1 = *(const v4f *)(kat + 8 * l + 4);
            for (int q = 1; q < a.np; ++q) {
                p0 += *(const v4f *)(kat + (size_t)q * a.pstride + 8 * l);
                p1 += *(const v4f *)(kat + (size_t)q * a.pstride + 8 * l + 4);
            }
            v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
            v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
        }
        double ss = 0.0;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (double)v[e] * (double)v[e];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        const float inv = 1.0f / sqrtf((float)(ss / (double)R) + a.eps);
        const v4i nw = *(const v4i *)(a.norm + 8 * l);
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const uint32_t u = (uint32_t)nw[e >> 1];
            uint16_t h0, l0, h1, l1;
            split_bf16((v[e] * inv) * __uint_as_float(u << 16), h0, l0);
            split_bf16((v[e + 1] * inv) * __uint_as_float(u & 0xffff0000u), h1, l1);
            hw[e >> 1] = pack2(h0, h1);
            lw[e >> 1] = pack2(l0, l1);
        }
        *(v4i *)(a.lath + (size_t)t * R + 8 * l) = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
        *(v4i *)(a.latl + (size_t)t * R + 8 * l) = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
        if (l < 32) {
            const float2 cs = a.cs[(size_t)t * 32 + l];
            float ev = kat[R + 2 * l], od = kat[R + 2 * l + 1];
            for (int q = 1; q < a.np; ++q) {
                ev += kat[(size_t)q * a.pstride + R + 2 * l];
                od += kat[(size_t)q * a.pstride + R + 2 * l + 1];
            }
            const float ec = ev * cs.x, os = od * cs.y, oc = od * cs.x, es = ev * cs.y;
            _Float16 h0, l0, h1, l1;
            split_f16(ec - os, h0, l0);
            split_f16(oc + es, h1, l1);
            rp[w][l] = h0;
            rp[w][32 + l] = h1;
            // dims DN + l (k-block 2p) and DN + 32 + l (2p + 1): group (l >> 3) & 3, element l & 7
            const int g8 = (l >> 3) & 3, e = l & 7;
            k8p[w][g8][e] = (uint8_t)f16_to_bf8(h0);
            k8p[w][g8][8 + e] = (uint8_t)f16_to_bf8(h1);
            k8p[w][4 + g8][e] = (uint8_t)bf8_lo_s11(l0);
            k8p[w][4 + g8][8 + e] = (uint8_t)bf8_lo_s11(l1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // lanes of part 0: 16 bytes of the fp16 hi row (dims DN + 8c ..); part 1: K8 slot c & 3 of
        // the hi (c < 4) or lo part
        const int part = (l >> 3) & 1, c = l & 7;
        const v4i rv = part ? *(const v4i *)k8p[w][c] : *(const v4i *)&rp[w][8 * c];
        uint8_t *dst = part ? a.k8 + (size_t)t * 384 + (c < 4 ? 0 : kK8Lo) + 16 * (4 * (a.DN >> 6) + (c & 3))
                            : (uint8_t *)(a.kh + (size_t)t * QD + a.DN + 8 * c);
        const size_t hs = part ? (size_t)a.Sp * 384 : (size_t)a.Sp * QD * sizeof(_Float16);
        for (int h = l >> 4; h < a.NH; h += 4) *(v4i *)(dst + h * hs) = rv;
        return;
    }
    auto kv = [&](int r) {
        float v = kat[r];
        for (int q = 1; q < a.np; ++q) v += kat[(size_t)q * a.pstride + r];
        return v;
    };
    double ss = 0.0;
    for (int r = l; r < R; r += 64) {
        const double v = (double)kv(r);
        ss += v * v;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float mean_sq = (float)(ss / (double)R);
    const float inv = 1.0f / sqrtf(mean_sq + a.eps);
    for (int r = l; r < R; r += 64) {
        const float v = kv(r) * inv;
        const float y = v * bf16_to_f32(a.norm[r]);
        uint16_t hh, ll;
        split_bf16(y, hh, ll);
        a.lath[(size_t)t * R + r] = hh;
        a.latl[(size_t)t * R + r] = ll;
    }
    for (int i = l; i < half; i += 64) {
        const float2 cs = a.cs[(size_t)t * half + i];
        const float ev = kv(R + 2 * i), od = kv(R + 2 * i + 1);
        const float ec = ev * cs.x, os = od * cs.y, oc = od * cs.x, es = ev * cs.y;
        _Float16 h0, l0, h1, l1;
        split_f16(ec - os, h0, l0);
        split_f16(oc + es, h1, l1);
        const int b0 = k8_hi_byte(a.DN + i), b1 = k8_hi_byte(a.DN + half + i);
        const uint8_t h0b = (uint8_t)f16_to_bf8(h0), l0b = (uint8_t)bf8_lo_s11(l0);
        const uint8_t h1b = (uint8_t)f16_to_bf8(h1), l1b = (uint8_t)bf8_lo_s11(l1);
        for (int h = 0; h < a.NH; ++h) {
            const size_t o = ((size_t)h * a.Sp + t) * QD + a.DN;
            uint8_t *row = a.k8 + ((size_t)h * a.Sp + t) * 384;
            a.kh[o + i] = h0;
            row[b0] = h0b;
            row[b0 + kK8Lo] = l0b;
            a.kh[o + half + i] = h1;
            row[b1] = h1b;
            row[b1 + kK8Lo] = l1b;
        }
    }
}

// ================================================================ flash attention ======

// Causal attention for one head and 128 queries: 4 waves x 32 queries (two 16-query tiles
// u = 0, 1), keys in tiles of 64. QD = 192, DV = 128. Operands are fp16 (11 significant bits,
// ample range for these values): Q and K as hi + lo pairs, V and P rounded once.
//
// Scores are computed transposed, S^T = K Q^T (A = K from LDS, B = Q^T from registers), as
// Kh Qh (v_mfma_f32_16x16x32_f16) plus the correction Kh Ql + Kl Qh as one bf8 product over
// 384 concatenated dims (v_mfma_scale_f32_16x16x128_f8f6f4, three per 16 x 16 tile): K8 rows
// hold bf8(Kh) and bf8(Kl 2^11) per lane group, the query operand bf8(Ql 2^11) and bf8(Qh) in
// the matching byte order, and the MFMA scales the product by 2^-11. The correction terms are
// 2^-11 of the product and bf8 keeps them to 2^-3, so the score error stays near 2^-14 of
// |K||Q| even for large logits, where a single rounding of K would be amplified by the logit
// size (the Kl Ql term is below 2^-22). Lane (g, n) then holds
// S^T[key 16t + 4g + i][query n], exactly the values it must supply as the B operand of
// O^T = V^T P^T when the k-slots of a 32-key chunk c are ordered (16-key tile 2c: i = 0..3,
// tile 2c+1: i = 0..3) per lane group g; V^T is stored with its keys permuted to that order
// (kv_b GEMM), so P never leaves the registers. Softmax is online with a lazy reference max
// per query: it moves only when a tile's max exceeds it by more than 8 (log2 units), so
// p <= 256 and most tiles skip the rescale.
//
// K and V tiles stream through LDS by global_load_lds_dwordx4 DMA into two offset rings:
// step j computes QK of tile j+1 (K ring) and softmax + PV of tile j (V ring) while K of
// tile j+2 and V of tile j+1 are in flight. The 16-byte slots of each LDS row are XOR-
// swizzled by the row so that the fragment reads are free of bank conflicts.
constexpr int kFQ = 128, kFK = 64;
constexpr int kFKB = kFK * 192 * 2;  // K tile (hi or lo): 64 rows x 384 B
constexpr int kFVB = 128 * kFK * 2;  // V^T tile: 128 rows x 128 B
constexpr int kFSmem = 2 * 2 * kFKB + 2 * kFVB;
constexpr float kFLazy = 8.0f;       // log2 headroom of the lazy max

struct FlashArgs {
    const _Float16 *qh, *kh;                 // Q, K hi: [NH, Sp, 192]
    const uint8_t *ql8;                      // bf8(Q lo x 2^11): [NH, Sp, 192]
    const uint8_t *k8;                       // K8 rows: [NH, Sp, 384 bytes]
    const _Float16 *vt;                      // V^T: [NH, 128, Sp]
    _Float16 *o;                             // [S, ldo] fp16 (input of the o_proj GEMM)
    int *flag_call, *flag_sticky;            // range flags (flag_sticky may be null)
    int S, Sp, NH, ldo;
    float sl2;                               // softmax scale * log2(e)
};

// Largest |row max logit| (natural units, scale included) for which the scores' bf8
// correction keeps the attention within the 2e-3 budget with margin: measured at 256 tokens,
// row-max logits up to ~150 give 3e-4, ~500 give 6e-4, ~1450 give 1.7e-3, ~4400 give 2.3e-3.
constexpr float kFLogitMax = 512.0f;

// Max / sum over the four lanes n, n + 16, n + 32, n + 48 (one per 16-lane row).
__device__ __forceinline__ float xrow_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float xrow_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_flash_prefill(FlashArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[kFSmem];
    const uint32_t sbase = lds_addr(smem);
    const int tid = threadIdx.x, l = tid & 63, n = l & 15, g = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // kernel arguments as locals (the lambdas below must not capture the argument block)
    const int S = a.S, Sp = a.Sp, NH = a.NH, ldo = a.ldo;
    const float sl2 = a.sl2;
    const int nqt = Sp / kFQ;
    // Longest tiles first; with NH % 8 == 0, block b runs on XCD b % 8 and each XCD keeps
    // the same NH / 8 heads, so the blocks streaming one head's K/V share an L2.
    int qt, h;
    if (NH % 8 == 0) {
        const int hpx = NH / 8, j = blockIdx.x >> 3;
        qt = nqt - 1 - j / hpx;
        h = (blockIdx.x & 7) + 8 * (j % hpx);
    } else {
        qt = nqt - 1 - (int)blockIdx.x / NH;
        h = (int)blockIdx.x % NH;
    }
    const int nt = 2 * qt + 2;  // key tiles 0 .. nt-1 (the last two straddle the diagonal)
    const int qw = qt * kFQ + 32 * w;
    const size_t hq = (size_t)h * Sp;

    // Q^T B operands: query qw + 16u + n, dims 32kb + 8g .. +7: hi as fp16 (main pass), lo as
    // its bf8(lo x 2^11) bytes (the correction operand below, written so by the q GEMM)
    v8h qa[2][6];
    uint2 qb[2][6];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const _Float16 *ph = a.qh + (hq + qw + 16 * u + n) * 192 + 8 * g;
        const uint8_t *pl = a.ql8 + (hq + qw + 16 * u + n) * 192 + 8 * g;
#pragma unroll
        for (int kb = 0; kb < 6; ++kb) {
            qa[u][kb] = *(const v8h *)(ph + 32 * kb);
            qb[u][kb] = *(const uint2 *)(pl + 32 * kb);
        }
    }

    // DMA sources. K tile: wave w fills LDS slots (6w + i) * 64 + l (16 B each) of the
    // 1536-slot tile; slot (row, s') holds logical slot s = s' ^ (row & 7) (within groups
    // of 8). V^T tile: slots (4w + i) * 64 + l of 1024; row d, slot s' holds s' ^ (d & 7).
    const uint8_t *gkh = (const uint8_t *)(a.kh + hq * 192);
    const uint8_t *gkl = a.k8 + hq * 384;
    const uint8_t *gv = (const uint8_t *)(a.vt + (size_t)h * 128 * Sp);
    uint32_t koff[6], voff[4];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int p = (6 * w + i) * 64 + l, row = p / 24, sp = p % 24;
        koff[i] = row * 384 + 16 * ((sp & ~7) | ((sp & 7) ^ (row & 7)));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = (4 * w + i) * 64 + l, d = p >> 3, sp = p & 7;
        voff[i] = (uint32_t)d * Sp * 2 + 16 * (sp ^ (d & 7));
    }
    // LDS: K ring [2][hi, lo], then V ring [2]
    auto issue_k = [&](int t) __attribute__((always_inline)) {
        const uint32_t dst = sbase + (t & 1) * 2 * kFKB + (uint32_t)(6 * w) * 1024;
        const size_t so = (size_t)t * kFK * 384;
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            dma_b128(gkh + so + koff[i], dst + i * 1024);
            dma_b128(gkl + so + koff[i], dst + kFKB + i * 1024);
        }
    };
    auto issue_v = [&](int t) __attribute__((always_inline)) {
        const uint32_t dst = sbase + 4 * kFKB + (t & 1) * kFVB + (uint32_t)(4 * w) * 1024;
#pragma unroll
        for (int i = 0; i < 4; ++i) dma_b128(gv + (size_t)t * 128 + voff[i], dst + i * 1024);
    };
    // LDS fragment offsets. K (A operand): row 16t + n, logical slot 4kb + g.
    // V^T (A operand): row 16dt + n, logical slot 4c + g.
    int krd[6], vrd[2];
#pragma unroll
    for (int kb = 0; kb < 6; ++kb) krd[kb] = n * 384 + 16 * (8 * (kb >> 1) + ((4 * (kb & 1) + g) ^ (n & 7)));
#pragma unroll
    for (int c = 0; c < 2; ++c) vrd[c] = n * 128 + 16 * ((4 * c + g) ^ (n & 7));
    // K8 (A operand of correction MFMA m): row 16t + n, logical slots 8m + g and 8m + 4 + g
    int f8rd[3][2];
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int ls = 8 * m + 4 * h2 + g;
            f8rd[m][h2] = n * 384 + 16 * ((ls & ~7) | ((ls & 7) ^ (n & 7)));
        }

    issue_k(0);
    issue_k(1);
    issue_v(0);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int kb = 0; kb < 6; ++kb) asm volatile("" : "+v"(qa[u][kb]), "+v"(qb[u][kb].x), "+v"(qb[u][kb].y));
    wait_vmcnt<0>();
    // correction operands: per u, 96 bytes = bf8(Ql 2^11) then bf8(Qh), each in (k-block,
    // element) order, so that byte p meets byte p of the lane group's K8 bytes (hi, then lo);
    // MFMA m takes bytes 32m .. 32m+31
    v8i q8[2][3];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        uint32_t wd[24];
#pragma unroll
        for (int kb = 0; kb < 6; ++kb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                uint32_t hi = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) hi |= f16_to_bf8(qa[u][kb][4 * hf + i]) << (8 * i);
                wd[2 * kb + hf] = hf == 0 ? qb[u][kb].x : qb[u][kb].y;
                wd[12 + 2 * kb + hf] = hi;
            }
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int j = 0; j < 8; ++j) q8[u][m][j] = (int)wd[8 * m + j];
    }
    // the query operands live in AGPRs (MFMA reads its A/B operands from either file), which
    // leaves the VGPRs to the score accumulators the softmax reads
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int kb = 0; kb < 6; ++kb) asm volatile("" : "+a"(qa[u][kb]));
#pragma unroll
        for (int m = 0; m < 3; ++m) asm volatile("" : "+a"(q8[u][m]));
    }
    lds_barrier();

    // Step j: QK of tile j+1 (unless it is the last step) with the softmax of tile j, the DMA
    // of K(j+2) and V(j+1), and the reads of tile j's V fragments spread over its MFMAs, then PV
    // of tile j. With one wave per SIMD, VALU, DMA-issue and LDS instructions run under the
    // MFMAs only when they are interleaved with them in the wave's instruction stream, so the
    // step is laid out as 18 groups of eight independent QK MFMAs (k-block kb, pass p) separated
    // by scheduling fences, each carrying its share of the other work, and the scheduler is asked
    // to alternate MFMAs and VALU within a group. Each QK accumulator receives its products in
    // the order Kh Qh for kb = 0 .. 5, then the corrections m = 0 .. 2.
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    v4f acc[8][2];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int u = 0; u < 2; ++u) acc[dt][u] = v4f{0.f, 0.f, 0.f, 0.f};

    v4f sc[4][2];
    auto load_kh = [&](const uint8_t *kt, int kb, v8h (&kh)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t) kh[t] = *(const v8h *)(kt + t * 16 * 384 + krd[kb]);
    };
    auto load_k8 = [&](const uint8_t *kt, int m, v8i (&k8)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const v4i x0 = *(const v4i *)(kt + kFKB + t * 16 * 384 + f8rd[m][0]);
            const v4i x1 = *(const v4i *)(kt + kFKB + t * 16 * 384 + f8rd[m][1]);
            k8[t] = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };
    auto qk_main = [&](v4f (&s)[4][2], const v8h (&kf)[4], int kb) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u) s[t][u] = mfma_f16(kf[t], qa[u][kb], s[t][u]);
    };
    auto qk_corr = [&](v4f (&s)[4][2], const v8i (&kf)[4], int m) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u) s[t][u] = mfma_bf8_s11(kf[t], q8[u][m], s[t][u]);
    };
    {  // QK of tile 0
        const uint8_t *kt = smem;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u) sc[t][u] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 6; ++kb) {
            v8h kh[4];
            load_kh(kt, kb, kh);
            qk_main(sc, kh, kb);
        }
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            v8i k8[4];
            load_k8(kt, m, k8);
            qk_corr(sc, k8, m);
        }
    }

    auto step = [&](auto mask_tag, auto next_tag, int j) __attribute__((always_inline)) {
        constexpr bool kMask = decltype(mask_tag)::value;
        constexpr bool kNext = decltype(next_tag)::value;
        wait_vmcnt<0>();
        lds_barrier();
        const bool dk = j + 2 < nt, dv = j + 1 < nt;
        const uint32_t kdst = sbase + (j & 1) * 2 * kFKB + (uint32_t)(6 * w) * 1024;  // K(j+2)
        const size_t kso = (size_t)(j + 2) * kFK * 384;
        const uint32_t vdst = sbase + 4 * kFKB + ((j + 1) & 1) * kFVB + (uint32_t)(4 * w) * 1024;  // V(j+1)
        auto dma_k = [&](int i) __attribute__((always_inline)) {
            if (dk) {
                dma_b128_s(gkh + kso, koff[i], kdst + i * 1024);
                dma_b128_s(gkl + kso, koff[i], kdst + kFKB + i * 1024);
            }
        };
        auto dma_v = [&](int i) __attribute__((always_inline)) {
            if (dv) dma_b128_s(gv + (size_t)(j + 1) * 128, voff[i], vdst + i * 1024);
        };
        // softmax of tile j in pieces (per 16-query tile u: A mask + local max, B row max and
        // reference max, C(t) weights of key tile t, D denominator)
        const int k0 = j * kFK;
        float mloc[2], mnew[2], alpha[2], ps[2];
        bool moved = false;
        v8h pb[2][2];
        auto smA = [&](int u) __attribute__((always_inline)) {
            const int q = qw + 16 * u + n;
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = sc[t][u][i];
                    if constexpr (kMask) {
                        const int key = k0 + 16 * t + 4 * g + i;
                        if (key > q || key >= S) v = -INFINITY;
                        sc[t][u][i] = v;
                    }
                    mx = fmaxf(mx, v);
                }
            mloc[u] = mx;
        };
        auto smB = [&](int u) __attribute__((always_inline)) {
            const float mx = xrow_max(mloc[u]) * sl2;
            const float mref = m_run[u];
            const bool mv = mx > mref + kFLazy;
            mnew[u] = mv ? mx : mref;
            alpha[u] = __builtin_amdgcn_exp2f(mref - mnew[u]);
            m_run[u] = mnew[u];
            moved |= mv;
            ps[u] = 0.f;
        };
        auto smC = [&](int u, int t) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = __builtin_amdgcn_exp2f(fmaf(sc[t][u][i], sl2, -mnew[u]));
                ps[u] += p;
                pb[u][t >> 1][4 * (t & 1) + i] = (_Float16)p;
            }
        };
        auto smD = [&](int u) __attribute__((always_inline)) { l_run[u] = fmaf(l_run[u], alpha[u], ps[u]); };
        // V fragments of tile j: row 16 dt + n, logical slot 4c + g
        const uint8_t *vt = smem + 4 * kFKB + (j & 1) * kFVB;
        v8h vv[2][8];
        auto load_v = [&](int f) __attribute__((always_inline)) {
            vv[f >> 3][f & 7] = *(const v8h *)(vt + (f & 7) * 16 * 128 + vrd[f >> 3]);
        };
        // the work carried by group gi (gi < 6: main pass kb = gi, eight MFMAs of 16 cycles;
        // gi = 6 .. 8: correction m = gi - 6, eight MFMAs of 32 cycles)
        auto extra = [&](int gi) __attribute__((always_inline)) {
            switch (gi) {
            case 0: smA(0); dma_k(0); dma_k(1); break;
            case 1: smB(0); dma_k(2); dma_k(3); break;
            case 2: smC(0, 0); smC(0, 1); dma_k(4); dma_k(5); break;
            case 3: smC(0, 2); smC(0, 3); smD(0); dma_v(0); dma_v(1); break;
            case 4: smA(1); dma_v(2); dma_v(3); break;
            case 5: smB(1); load_v(0); load_v(1); break;
            case 6: smC(1, 0); smC(1, 1); load_v(2); load_v(3); load_v(4); load_v(5); break;
            case 7: smC(1, 2); smC(1, 3); smD(1); load_v(6); load_v(7); load_v(8); load_v(9); break;
            case 8: load_v(10); load_v(11); load_v(12); load_v(13); load_v(14); load_v(15); break;
            default: break;
            }
        };
        if constexpr (kNext) {
            const uint8_t *kt = smem + ((j + 1) & 1) * 2 * kFKB;  // K tile j+1
            v4f sn[4][2];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int u = 0; u < 2; ++u) sn[t][u] = v4f{0.f, 0.f, 0.f, 0.f};
            v8h kh[2][4];
            v8i k8[2][4];
            load_kh(kt, 0, kh[0]);
#pragma unroll
            for (int kb = 0; kb < 6; ++kb) {
                const int cb = kb & 1;
                if (kb + 1 < 6) load_kh(kt, kb + 1, kh[cb ^ 1]);
                if (kb == 4) load_k8(kt, 0, k8[0]);
                if (kb == 5) load_k8(kt, 1, k8[1]);
                __builtin_amdgcn_sched_barrier(0);
                qk_main(sn, kh[cb], kb);
                extra(kb);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // up to three VALU
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                if (m == 1) load_k8(kt, 2, k8[0]);  // k8[0] is free once correction 0 has issued
                __builtin_amdgcn_sched_barrier(0);
                qk_corr(sn, k8[m & 1], m);
                extra(6 + m);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // up to six VALU
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            // the softmax results stay in the groups above (the compiler would otherwise sink
            // them past the rescale branch, to their uses)
            asm volatile("" ::"v"(pb[0][0]), "v"(pb[0][1]), "v"(pb[1][0]), "v"(pb[1][1]), "v"(l_run[0]),
                         "v"(l_run[1]));
            const bool any = __any(moved);
            if (any) {
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                    for (int u = 0; u < 2; ++u) acc[dt][u] *= alpha[u];
            }
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                    for (int u = 0; u < 2; ++u) acc[dt][u] = mfma_f16(vv[c][dt], pb[u][c], acc[dt][u]);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int u = 0; u < 2; ++u) sc[t][u] = sn[t][u];
        } else {
#pragma unroll
            for (int gi = 0; gi < 9; ++gi) extra(gi);
            if (__any(moved)) {
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                    for (int u = 0; u < 2; ++u) acc[dt][u] *= alpha[u];
            }
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                    for (int u = 0; u < 2; ++u) acc[dt][u] = mfma_f16(vv[c][dt], pb[u][c], acc[dt][u]);
        }
    };
    using F = std::false_type;
    using T = std::true_type;
    for (int j = 0; j < nt - 2; ++j) step(F{}, T{}, j);
    step(T{}, T{}, nt - 2);
    step(T{}, F{}, nt - 1);

    // range check of each query row: the reference max m_run (log2 units, within kFLazy of the
    // row's true max) and every output value (NaN or Inf from operands beyond the fp16 range)
    bool bad = false;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int q = qw + 16 * u + n;
        const float inv = 1.0f / xrow_sum(l_run[u]);
        if (q >= S) continue;
        bad |= !(fabsf(m_run[u]) <= kFLogitMax * 1.4426950408889634f);  // m_run = logit * log2(e)
        _Float16 *o = a.o + (size_t)q * ldo + (size_t)h * 128 + 4 * g;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const v4h ov = {(_Float16)(acc[dt][u][0] * inv), (_Float16)(acc[dt][u][1] * inv),
                            (_Float16)(acc[dt][u][2] * inv), (_Float16)(acc[dt][u][3] * inv)};
#pragma unroll
            for (int i = 0; i < 4; ++i) bad |= !__builtin_isfinite((float)ov[i]);
            *(v4h *)(o + 16 * dt) = ov;
        }
    }
    // any writer stores the same value; the readers are later kernels
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && l == 0) {
        __hip_atomic_store(a.flag_call, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (a.flag_sticky) __hip_atomic_store(a.flag_sticky, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
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
// Queries t0 .. t0 + gridDim.x - 1 (one tile of the sequence: the score scratch holds one row
// of S scores per (query of the tile, head), so its size stays linear in S).
struct GenAttnArgs {
    const float *qf, *kv, *krope;
    float *heads, *scr;
    int S, NH, DN, DR, DV, t0;
    float smscale;
};

__global__ __launch_bounds__(256) void k_gen_attn(GenAttnArgs a) {
    __shared__ float red[256];
    const int t = a.t0 + blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int QD = a.DN + a.DR, KH = a.DN + a.DV, L = t + 1;
    const float *q = a.qf + ((size_t)t * a.NH + h) * QD;
    float *sc = a.scr + ((size_t)blockIdx.x * a.NH + h) * a.S;
    for (int j = tid; j < L; j += 256) {
        const float *kj = a.kv + (size_t)j * a.NH * KH + (size_t)h * KH;
        const float *rj = a.krope + (size_t)j * a.DR;
        // the dots in double and the score as (float)dot * scale, as
        // src/mla_prefill_streaming.c:171-174
        double acc = 0.0;
        for (int k = 0; k < a.DN; ++k) acc = fma((double)q[k], (double)kj[k], acc);
        for (int k = 0; k < a.DR; ++k) acc = fma((double)q[a.DN + k], (double)rj[k], acc);
        sc[j] = (float)acc * a.smscale;
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

__global__ __launch_bounds__(256) void k_bf16_to_f16(_Float16 *dst, const uint16_t *src, size_t n, float scale) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = (_Float16)(bf16_to_f32(src[i]) * scale);
}

hipError_t launch_split(hipStream_t st, const float *src, int ld_src, uint16_t *hi, uint16_t *lo,
                        int ld_dst, int rows, int cols) {
    if (rows < 1 || cols < 8 || cols % 8 || ld_src % 4 || ld_dst % 8 || ld_src < cols || ld_dst < cols ||
        ((uintptr_t)src % 16) || ((uintptr_t)hi % 16) || ((uintptr_t)lo % 16))
        return hipErrorInvalidValue;
    const int blocks = std::min(2048, rows);  // k_split loops over rows by block
    hipLaunchKernelGGL(k_split, dim3(blocks), dim3(256), 0, st, src, ld_src, hi, lo, ld_dst, rows, cols,
                       nullptr);
    return hipGetLastError();
}

hipError_t launch_bf16_to_f16(hipStream_t st, _Float16 *dst, const uint16_t *src, size_t n, float scale) {
    const int blocks = (int)std::min<size_t>(4096, (n + 255) / 256);
    hipLaunchKernelGGL(k_bf16_to_f16, dim3(blocks), dim3(256), 0, st, dst, src, n, scale);
    return hipGetLastError();
}

bool prefill_mfma_shape(const Dims &d) {
    return d.H % 64 == 0 && d.R % 64 == 0 && d.QD == 192 && d.DV == 128 && d.HO % 64 == 0 &&
           d.DN % 8 == 0;
}

bool prefill_kva_exact(const Dims &d) { return prefill_mfma_shape(d) && gemv_ksplit_ok(d.H, d.H); }

// Queries per launch of the generic route's attention: the score scratch (queries x NH x S
// fp32) stays within 64 MiB, or one query's NH x S when that alone is larger.
static int gen_query_tile(const Dims &d, int S) {
    const size_t per_query = (size_t)d.NH * (size_t)S;
    const size_t cap = (size_t)16 << 20;  // floats
    return (int)std::max<size_t>(1, std::min<size_t>((size_t)S, cap / per_query));
}

size_t prefill_bytes(const Dims &d, int S, bool generic) {
    const size_t Sp = (size_t)(S + 127) / 128 * 128;
    size_t b = 0;
    auto add = [&](size_t n) { b += (n + 255) / 256 * 256 + 256; };
    if (prefill_mfma_shape(d) && !generic) {
        add(4 * 8);                              // flags
        add(2 * (size_t)S * d.H);                // x hi
        add(2 * (size_t)S * d.H);                // x lo
        add(4 * (size_t)S * d.KVO * (prefill_kva_exact(d) ? kGemvKs : 1));  // kv_a projection
        add(2 * (size_t)S * d.R);                // latent hi
        add(2 * (size_t)S * d.R);                // latent lo
        add(2 * (size_t)d.NH * Sp * d.QD);       // q hi (fp16)
        add(2 * (size_t)d.NH * Sp * d.QD);       // q lo
        add(2 * (size_t)d.NH * Sp * d.QD);       // k hi
        add(2 * (size_t)d.NH * Sp * d.QD);       // k lo
        add(2 * (size_t)d.NH * d.DV * Sp);       // v^T
        add(2 * (size_t)S * d.HO);               // heads (fp16)
    } else {
        add(4 * (size_t)S * (d.QO + d.KVO));
        add(4 * (size_t)S * d.R);
        add(4 * (size_t)S * d.DR);
        add(4 * (size_t)S * d.NH * d.QD);
        add(4 * (size_t)S * d.KVB);
        add(4 * (size_t)S * d.HO);
        add(4 * (size_t)gen_query_tile(d, S) * d.NH * S);
    }
    return b;
}

hipError_t launch_prefill_all(hipStream_t st, const Dims &d, int S, float eps, const float *x,
                              float *out, const uint16_t *wq, const uint16_t *wkva,
                              const uint16_t *wnorm, const uint16_t *wkvb, const uint16_t *wo,
                              const _Float16 *wo16, const float2 *cs, void *ws, PrefillKva *kva,
                              const PrefillRange *range) {
    const int Sp = (S + 127) / 128 * 128;
    if (kva) *kva = PrefillKva{nullptr, 0, 0, 0};
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
    if (prefill_mfma_shape(d) && !(range && range->generic)) {
        int *flags = (int *)take(4 * 8);
        uint16_t *xh = (uint16_t *)take(2 * (size_t)S * d.H);
        uint16_t *xl = (uint16_t *)take(2 * (size_t)S * d.H);
        const bool exact = kva && prefill_kva_exact(d);
        const int np = exact ? kGemvKs : 1;
        float *ykva = (float *)take(4 * (size_t)S * d.KVO * np);
        uint16_t *lath = (uint16_t *)take(2 * (size_t)S * d.R);
        uint16_t *latl = (uint16_t *)take(2 * (size_t)S * d.R);
        _Float16 *qh = (_Float16 *)take(2 * (size_t)d.NH * Sp * d.QD);
        uint8_t *ql8 = (uint8_t *)take((size_t)d.NH * Sp * d.QD);
        _Float16 *kh = (_Float16 *)take(2 * (size_t)d.NH * Sp * d.QD);
        uint8_t *k8 = (uint8_t *)take((size_t)d.NH * Sp * 384);
        _Float16 *vt = (_Float16 *)take(2 * (size_t)d.NH * d.DV * Sp);
        _Float16 *heads = (_Float16 *)take(2 * (size_t)S * d.HO);
        GemmEpi ep{qh, kh, ql8, k8, vt, cs, Sp, d.DN, d.DR, d.DV};
        const float vscale = range ? range->vscale : 1.0f, oscale = range ? range->oscale : 1.0f;
        // flags[0] (any x lo word non-zero) is raised by k_split and cleared by k_kva_pack after
        // the q GEMM has read it, so no launch clears it first. A value left raised (a call
        // that failed in between, or the buffer reused by another call) only costs the GEMM's lo
        // pass over an exact plane: the flag is never clear while a lo word is non-zero.
        const int split_blocks = std::min(2048, S);
        hipLaunchKernelGGL(k_split, dim3(split_blocks), dim3(256), 0, st, x, d.H, xh, xl, d.H, S, d.H, flags + 0);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // q (-> Q hi/lo, rotated) | kv_a (-> ykva). When the caller fills a state from this
        // kv_a, it is computed with the decode's k-split arithmetic (launch_kva_tok) so those
        // rows equal the rows a decode appends; otherwise it rides along in the q GEMM.
        if (exact) {
            if ((e = gemm<kEpiQ>(st, xh, xl, flags + 0, d.H, wq, d.QO, nullptr, 0, d.H, nullptr, 0, S, d.H,
                                 ep)) != hipSuccess)
                return e;
            if ((e = launch_kva_tok(st, ykva, (size_t)S * d.KVO, d.KVO, xh, xl, S, wkva, d.KVO, d.H)) !=
                hipSuccess)
                return e;
            if (kva) *kva = PrefillKva{ykva, d.KVO, np, (size_t)S * d.KVO};
        } else if ((e = gemm<kEpiQ>(st, xh, xl, flags + 0, d.H, wq, d.QO, wkva, d.KVO, d.H, ykva, d.KVO, S,
                                    d.H, ep)) != hipSuccess) {
            return e;
        }
        KvaPackArgs ka{ykva, wnorm, cs, lath, latl, qh, ql8, kh, k8, vt, (size_t)S * d.KVO, np,
                       S, Sp, d.NH, d.KVO, d.R, d.DN, d.DR, d.DV, eps, flags + 0};
        hipLaunchKernelGGL(k_kva_pack, dim3((Sp + 3) / 4), dim3(256), 0, st, ka);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // kv_b (-> K nope part as fp16 hi + K8, V^T scaled by vscale)
        ep.vscale = vscale;
        if ((e = gemm<kEpiKV>(st, lath, latl, nullptr, d.R, wkvb, d.KVB, nullptr, 0, d.R, nullptr, 0, S, d.R,
                              ep)) != hipSuccess)
            return e;
        FlashArgs fa{qh, kh, ql8, k8, vt, heads, flags + 1, range ? range->sticky : nullptr, S, Sp, d.NH, d.HO,
                     smscale * 1.4426950408889634f};
        hipLaunchKernelGGL(k_flash_prefill, dim3(Sp / kFQ * d.NH), dim3(256), 0, st, fa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // out = heads . o_proj^T in fp16 (heads rounded once, o_proj converted exactly), the
        // two scales undone (or NaN when the range flag of this call is up)
        if (!wo16) return hipErrorInvalidValue;
        ep.vscale = 1.0f;
        ep.alpha = 1.0f / (vscale * oscale);
        ep.nan_flag = flags + 1;
        return gemm<kEpiPlain, true>(st, (const uint16_t *)heads, nullptr, nullptr, d.HO, (const uint16_t *)wo16, d.H,
                                     nullptr, 0, d.HO, out, d.H, S, d.HO, ep);
    }
    float *y = (float *)take(4 * (size_t)S * ldy);
    float *latf = (float *)take(4 * (size_t)S * d.R);
    float *krope = (float *)take(4 * (size_t)S * d.DR);
    float *qf = (float *)take(4 * (size_t)S * d.NH * d.QD);
    float *kv = (float *)take(4 * (size_t)S * d.KVB);
    float *heads = (float *)take(4 * (size_t)S * d.HO);
    const int tq = gen_query_tile(d, S);
    float *scr = (float *)take(4 * (size_t)tq * d.NH * S);
    if ((e = launch_gemv(st, y, ldy, x, d.H, S, wq, d.QO, wkva, d.KVO, d.H, false)) != hipSuccess) return e;
    KvaEpiArgs ea{y, wnorm, cs, latf, nullptr, nullptr, krope, nullptr, ldy, d.QO, d.R, d.DR, eps};
    hipLaunchKernelGGL(k_kva_epi, dim3(S), dim3(256), 0, st, ea);
    GenEpiArgs ga{y, wnorm, cs, latf, krope, qf, ldy, d.NH, d.DN, d.DR, d.R, d.QO, eps};
    hipLaunchKernelGGL(k_gen_epi, dim3(S), dim3(256), 0, st, ga);
    if ((e = launch_gemv(st, kv, d.KVB, latf, d.R, S, wkvb, d.KVB, nullptr, 0, d.R, false)) != hipSuccess)
        return e;
    for (int t0 = 0; t0 < S; t0 += tq) {
        GenAttnArgs aa{qf, kv, krope, heads, scr, S, d.NH, d.DN, d.DR, d.DV, t0, smscale};
        hipLaunchKernelGGL(k_gen_attn, dim3(std::min(tq, S - t0), d.NH), dim3(256), 0, st, aa);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return launch_gemv(st, out, d.H, heads, d.HO, S, wo, d.H, nullptr, 0, d.HO, false);
}

}  // namespace kvl
