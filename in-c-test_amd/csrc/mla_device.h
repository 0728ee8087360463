// Device helpers shared by the MLA kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvl {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

// Round-to-nearest-even with the history format's rule: Inf/NaN words are truncated,
// NaN payloads kept (src/mla_compressed_q8_state.c:9-16).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) != 0x7f800000u) u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// x ~= hi + lo with hi, lo bf16: the split keeps ~16 mantissa bits of an fp32 operand
// for bf16 MFMA (products with bf16-exact operands stay exact in the fp32 accumulator).
__device__ __forceinline__ void split_bf16(float x, uint16_t &hi, uint16_t &lo) {
    hi = f32_to_bf16_rne(x);
    lo = f32_to_bf16_rne(x - bf16_to_f32(hi));
}

__device__ __forceinline__ uint32_t pack2(uint16_t a, uint16_t b) {
    return (uint32_t)a | ((uint32_t)b << 16);
}

// 8 fp32 values -> two bf16x8 MFMA operands (hi, lo).
__device__ __forceinline__ void split8(const v4f &x0, const v4f &x1, v8bf &hi, v8bf &lo) {
    uint16_t h[8], l[8];
    split_bf16(x0.x, h[0], l[0]);
    split_bf16(x0.y, h[1], l[1]);
    split_bf16(x0.z, h[2], l[2]);
    split_bf16(x0.w, h[3], l[3]);
    split_bf16(x1.x, h[4], l[4]);
    split_bf16(x1.y, h[5], l[5]);
    split_bf16(x1.z, h[6], l[6]);
    split_bf16(x1.w, h[7], l[7]);
    v4i hv = {(int)pack2(h[0], h[1]), (int)pack2(h[2], h[3]), (int)pack2(h[4], h[5]),
              (int)pack2(h[6], h[7])};
    v4i lv = {(int)pack2(l[0], l[1]), (int)pack2(l[2], l[3]), (int)pack2(l[4], l[5]),
              (int)pack2(l[6], l[7])};
    hi = __builtin_bit_cast(v8bf, hv);
    lo = __builtin_bit_cast(v8bf, lv);
}

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// split8 with the hardware conversion (v_cvt_pk_bf16_f32: round to nearest even, one instruction
// per pair): hi = bf16(x), lo = bf16(x - hi), x - hi being exact. For finite values the same
// words as split8, in about a fifth of the VALU instructions.
__device__ __forceinline__ void split8_cvt(const v4f &x0, const v4f &x1, v8bf &hi, v8bf &lo) {
    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    v2bf h[4], l[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const v2f xp = {x[2 * p], x[2 * p + 1]};
        h[p] = __builtin_convertvector(xp, v2bf);
        const v2f hf = {(float)h[p].x, (float)h[p].y};
        const v2f r = {xp.x - hf.x, xp.y - hf.y};
        l[p] = __builtin_convertvector(r, v2bf);
    }
    hi = __builtin_shufflevector(__builtin_shufflevector(h[0], h[1], 0, 1, 2, 3),
                                 __builtin_shufflevector(h[2], h[3], 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
    lo = __builtin_shufflevector(__builtin_shufflevector(l[0], l[1], 0, 1, 2, 3),
                                 __builtin_shufflevector(l[2], l[3], 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
}

// One half of the split x ~= hi + lo of 8 fp32 values as a bf16x8 MFMA operand: part 0 the hi
// halves, part 1 the lo halves (both round to nearest even, v_cvt_pk_bf16_f32). Finite inputs.
__device__ __forceinline__ v8bf split8_part(const v4f &x0, const v4f &x1, int part) {
    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    v4i o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const v2f p = {x[2 * j], x[2 * j + 1]};
        const uint32_t hu = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, v2bf));
        const v2f r = {x[2 * j] - __uint_as_float(hu << 16), x[2 * j + 1] - __uint_as_float(hu & 0xffff0000u)};
        const uint32_t lu = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, v2bf));
        o[j] = (int)(part ? lu : hu);
    }
    return __builtin_bit_cast(v8bf, o);
}

__device__ __forceinline__ v4f mfma_bf16(const v8bf &a, const v8bf &b, const v4f &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_f16(const v8h &a, const v8h &b, const v4f &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// C += (A x 2^-11) . B with A, B bf8 (e5m2) operands, 16 x 16 x 128 (E8M0 scales 116 and 127).
// Lane (row or column c, group g) holds 32 bytes; byte p of A lane (r, g) multiplies byte p of
// B lane (c, g), and the result has the layout of mfma_f16.
__device__ __forceinline__ v4f mfma_bf8_s11(const v8i &a, const v8i &b, const v4f &c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 1, 1, 0, 116, 0, 127);
}

// bf8 (e5m2: the sign, exponent and top two mantissa bits of fp16) of an fp16 value, rounded to
// nearest with ties away from zero, saturating at +-57344.
__device__ __forceinline__ uint32_t f16_to_bf8(_Float16 x) {
    const uint32_t h = __builtin_bit_cast(uint16_t, x), m = h & 0x7fffu;
    return ((h >> 8) & 0x80u) | (m > 0x7b7fu ? 0x7bu : (m + 0x80u) >> 8);
}

// K8 row (384 bytes) of a key: 24 slots of 16 bytes, slot (part, k-block pair p, lane group g)
// at 12 part + 4 p + g holding the bf8 of dims 32 kb + 8 g + e for kb = 2p, 2p + 1, e = 0 .. 7 in
// that order: part 0 the fp16 hi parts, part 1 the lo parts x 2^11 (kK8Lo bytes further). A
// lane of group g reads its 96-byte correction operand as slots 4j + g, j = 0 .. 5, and 16
// lanes writing 64 consecutive dims write 64 contiguous bytes of each part.
constexpr int kK8Lo = 192;
__device__ __forceinline__ int k8_hi_byte(int d) {
    return 16 * (4 * (d >> 6) + ((d >> 3) & 3)) + 8 * ((d >> 5) & 1) + (d & 7);
}
__device__ __forceinline__ uint32_t bf8_lo_s11(_Float16 lo) { return f16_to_bf8((_Float16)((float)lo * 2048.0f)); }

// x ~= hi + lo with hi, lo fp16 (round to nearest even): the split keeps ~22 mantissa bits of
// an fp32 operand of moderate range; products of fp16 operands are exact in fp32.
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}
__device__ __forceinline__ void split8_f16(const float *x, v8h &hi, v8h &lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        _Float16 h, l;
        split_f16(x[i], h, l);
        hi[i] = h;
        lo[i] = l;
    }
}
__device__ __forceinline__ v4i mfma_i8(const v4i &a, const v4i &b, const v4i &c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Reductions over the 16 lanes of each DPP row (lanes 16r .. 16r+15) with DPP moves:
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror:4, row_ror:8.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x124>(v));
    v = fmaxf(v, dpp_f32<0x128>(v));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x124>(v);
    v += dpp_f32<0x128>(v);
    return v;
}

// Reductions over the whole (fully active) wave: DPP within each row of 16 lanes, then the
// four row results read as scalars (the result is wave-uniform).
__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double lane_f64(double v, int lane) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<0xB1>(v);
    v += dpp_f64<0x4E>(v);
    v += dpp_f64<0x124>(v);
    v += dpp_f64<0x128>(v);
    return (lane_f64(v, 0) + lane_f64(v, 16)) + (lane_f64(v, 32) + lane_f64(v, 48));
}
// Max / sum over a workgroup of 256 threads (four full waves): wave reductions, then the four
// wave results through `red4` (4 LDS entries, used once per call site) and one barrier.
__device__ __forceinline__ float block256_max(float v, float *red4) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
}
__device__ __forceinline__ double block256_sum_f64(double v, double *red4) {
    v = wave_sum_f64(v);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)p; }

// Asynchronous global -> LDS copies: lane l's bytes land at lds_base + l * size. lds_base
// must be wave-uniform. M0 is saved and restored around the instruction. GFX9 needs one
// wait state between an SALU write of M0 and a global load with LDS = 1 that reads it; the
// compiler inserts it for its own code but not inside an asm statement, hence the s_nop.
__device__ __forceinline__ void dma_b128(const void *gptr, uint32_t lds_base) {
    lds_base = __builtin_amdgcn_readfirstlane(lds_base);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(lds_base), "v"(gptr)
                 : "memory");
}
// The same copy with the non-temporal hint, for streams read once (a decode's history rows):
// measured 5.4 -> 5.7-5.8 TB/s for a 1 GiB streaming read with plain loads, and 7 % less time
// for the Q8 attention of 8 x 32K rows; the caches are not filled with data never read again.
__device__ __forceinline__ void dma_b128_nt(const void *gptr, uint32_t lds_base) {
    lds_base = __builtin_amdgcn_readfirstlane(lds_base);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off nt\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(lds_base), "v"(gptr)
                 : "memory");
}
// The same copy with the address as a wave-uniform 64-bit base (SGPRs) plus a per-lane 32-bit
// byte offset: no 64-bit VALU address add per instruction.
__device__ __forceinline__ void dma_b128_s(const void *sbase, uint32_t voff, uint32_t lds_base) {
    lds_base = __builtin_amdgcn_readfirstlane(lds_base);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(lds_base), "v"(voff), "s"(sbase)
                 : "memory");
}
__device__ __forceinline__ void dma_b32(const void *gptr, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(lds_base), "v"(gptr)
                 : "memory");
}
__device__ __forceinline__ void dma_b32_nt(const void *gptr, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, off nt\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(lds_base), "v"(gptr)
                 : "memory");
}
// History rows of a decode: non-temporal when each row is read by one workgroup (`once`),
// cached when the members of a block launch read the same rows at about the same time on one
// XCD (its L2 then serves the later members). `once` is wave-uniform.
__device__ __forceinline__ void dma_hist_b128(const void *gptr, uint32_t lds_base, bool once) {
    if (once) dma_b128_nt(gptr, lds_base);
    else dma_b128(gptr, lds_base);
}
__device__ __forceinline__ void dma_hist_b32(const void *gptr, uint32_t lds_base, bool once) {
    if (once) dma_b32_nt(gptr, lds_base);
    else dma_b32(gptr, lds_base);
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier after this wave's LDS writes have completed.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// SplitMix64 output k (k >= 1) of the stream seeded by `seed`.
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t k) {
    uint64_t z = seed + k * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Approximately N(0,1): Irwin-Hall sum of four 24-bit uniforms, centred and scaled by
// sqrt(3). Only exactly rounded fp32 operations, so a host mirror reproduces it bit for bit.
__device__ __forceinline__ float synth_normal(uint64_t seed, uint64_t idx) {
    float u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        u[k] = (float)(uint32_t)(splitmix64_at(seed, 4 * idx + k + 1) >> 40) * 5.9604644775390625e-8f;
    const float s = (u[0] + u[1]) + (u[2] + u[3]);
    return (s - 2.0f) * 1.7320508f;
}

}  // namespace kvl
