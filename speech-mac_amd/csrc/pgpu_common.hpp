// Shared device helpers for the gfx950 decode-step kernels.
//
// Activation operands of the projections are kept in "split fragment" form:
// every fp32 activation x is written as three bf16 terms hi + mid + lo that
// sum to x exactly (truncation split: hi keeps the top 8 significand bits,
// mid the next 8, lo the remaining <= 8), laid out in the operand order of
// v_mfma_f32_16x16x32_bf16 so that one lane's B operand is 16 contiguous
// bytes. With int8 (or bf16) weights every MFMA product is exact in fp32, so
// three bf16 MFMAs reproduce an fp32 dot product to fp32 accumulation error.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "phonon_gpu.h"

extern "C" void pgpu_record_error(const char *what);

namespace pgpu {

// Launch bookkeeping of the C-ABI launchers: 1 on success, else 0 with the
// reason kept for pgpu_last_error().
inline int launch_ok(const char *name) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return 1;
    char text[256];
    snprintf(text, sizeof(text), "%s: launch failed: %s", name, hipGetErrorString(e));
    pgpu_record_error(text);
    return 0;
}

inline int bad_arguments(const char *name) {
    char text[256];
    snprintf(text, sizeof(text), "%s: invalid arguments", name);
    pgpu_record_error(text);
    return 0;
}

constexpr int kWidth = 512;      // model width D
constexpr int kHeads = 8;        // attention heads
constexpr int kHeadDim = 64;     // head width
constexpr int kFfn = 2048;       // MLP width
constexpr int kBlockPos = 16;    // positions per KV block
constexpr int kSplitKeys = 256;  // keys per attention work-group (16 blocks)
constexpr int kMaxPositions = 8192;

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// Split formats (the `terms` of a split-fragment buffer): 3 bf16 terms
// (exact), the first 2 of them, or kF16Pair: two fp16 terms in the first two
// records (split2h).
constexpr int kF16Pair = PGPU_SPLIT_F16_PAIR;
__host__ __device__ constexpr int split_records(int terms) { return terms == kF16Pair ? 2 : terms; }

// Index (in bf16 elements) of activation x[s][k], part p (0 hi, 1 mid, 2 lo),
// inside a split-fragment buffer whose rows have kb_count 32-wide blocks.
// Record (stream tile st, block kb, part p) holds 64 lanes x 8 bf16; lane
// g*16 + n carries stream st*16+n, columns kb*32 + g*8 .. +7.
__host__ __device__ inline size_t split_index(int s, int k, int p, int kb_count) {
    const int st = s >> 4, n = s & 15, kb = k >> 5, g = (k >> 3) & 3, j = k & 7;
    return ((size_t)(st * kb_count + kb) * 3 + p) * 512 + (size_t)(g * 16 + n) * 8 + j;
}

__device__ inline uint32_t fbits(float x) { return __float_as_uint(x); }
__device__ inline float bitsf(uint32_t u) { return __uint_as_float(u); }

// Exact three-term truncation split; returns the bf16 bit patterns.
__device__ inline void split3(float x, uint16_t &hi, uint16_t &mid, uint16_t &lo) {
    const uint32_t h = fbits(x) & 0xffff0000u;
    const float r1 = __fsub_rn(x, bitsf(h));
    const uint32_t m = fbits(r1) & 0xffff0000u;
    const float r2 = __fsub_rn(r1, bitsf(m));
    hi = (uint16_t)(h >> 16);
    mid = (uint16_t)(m >> 16);
    lo = (uint16_t)(fbits(r2) >> 16);
}

// Two-term fp16 split: hi = fp16(x) (round to nearest), lo = fp16(x - hi);
// x - hi is exact in fp32, so hi + lo carries 22 significant bits of x
// while |x| stays inside the fp16 range (beyond 65504, hi is infinite and
// the products become non-finite, which the consumers flag); below 2^-14
// the terms lose bits to fp16 subnormals (absolute error under 2^-25).
__device__ inline void split2h(float x, uint16_t &hi, uint16_t &lo) {
    const _Float16 h = (_Float16)x;
    const _Float16 l = (_Float16)__fsub_rn(x, (float)h);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, l);
}

// Writes n (n = 4 or 8) consecutive activations of one stream starting at a
// column k that is a multiple of n, as three contiguous n*2-byte stores.
template <int N>
__device__ inline void store_split(uint16_t *__restrict__ xs, int s, int k, int kb_count,
                                   const float *v) {
    uint16_t h[N], m[N], l[N];
#pragma unroll
    for (int i = 0; i < N; i++) split3(v[i], h[i], m[i], l[i]);
    const size_t base = split_index(s, k, 0, kb_count);
    if constexpr (N == 8) {
        uint4 a, b, c;
        a.x = h[0] | (uint32_t)h[1] << 16; a.y = h[2] | (uint32_t)h[3] << 16;
        a.z = h[4] | (uint32_t)h[5] << 16; a.w = h[6] | (uint32_t)h[7] << 16;
        b.x = m[0] | (uint32_t)m[1] << 16; b.y = m[2] | (uint32_t)m[3] << 16;
        b.z = m[4] | (uint32_t)m[5] << 16; b.w = m[6] | (uint32_t)m[7] << 16;
        c.x = l[0] | (uint32_t)l[1] << 16; c.y = l[2] | (uint32_t)l[3] << 16;
        c.z = l[4] | (uint32_t)l[5] << 16; c.w = l[6] | (uint32_t)l[7] << 16;
        *(uint4 *)(xs + base) = a;
        *(uint4 *)(xs + base + 512) = b;
        *(uint4 *)(xs + base + 1024) = c;
    } else {
        static_assert(N == 4, "4 or 8 columns");
        uint2 a, b, c;
        a.x = h[0] | (uint32_t)h[1] << 16; a.y = h[2] | (uint32_t)h[3] << 16;
        b.x = m[0] | (uint32_t)m[1] << 16; b.y = m[2] | (uint32_t)m[3] << 16;
        c.x = l[0] | (uint32_t)l[1] << 16; c.y = l[2] | (uint32_t)l[3] << 16;
        *(uint2 *)(xs + base) = a;
        *(uint2 *)(xs + base + 512) = b;
        *(uint2 *)(xs + base + 1024) = c;
    }
}

// Sum over each row of 16 lanes (DPP row rotations, then quad permutes; no
// LDS traffic). Every lane of a row gets the same bits.
__device__ inline float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                0x128, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                0x124, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                0x4E, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                0xB1, 0xf, 0xf, false));
    return v;
}

// v + (v of the lane 16 apart within each half-wave), then + (the same of
// the lane 32 apart): the bits of v += shfl_xor(v, 16); v += shfl_xor(v, 32)
// (IEEE addition commutes), with gfx950's VALU lane swaps instead of LDS
// permutes. v_permlane16_swap(v, v) leaves rows (0, 0, 2, 2) in the first
// result and (1, 1, 3, 3) in the second; v_permlane32_swap(v, v) leaves the
// low half twice in the first and the high half twice in the second.
__device__ inline float xor16_32_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ inline float xor16_32_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Records a non-finite result: one atomic per wave at most.
__device__ inline void flag_nonfinite(int *status, bool bad) {
    if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(status, 1);
}

// A&S 7.1.26 erf with the fmaf chain of the reference's Torch-NEON
// adaptation (src/phonon_transformer.c:190-200); exp from the device libm.
__device__ inline float erf_as7126(float x) {
    const float t = 1.0f / fmaf(0.3275911f, fabsf(x), 1.0f);
    float r = fmaf(1.061405429f, t, -1.453152027f);
    r = fmaf(r, t, 1.421413741f);
    r = fmaf(r, t, -0.284496736f);
    r = fmaf(r, t, 0.254829592f);
    const float neg_exp = -expf(-__fmul_rn(x, x));
    return copysignf(fmaf(__fmul_rn(t, neg_exp), r, 1.0f), x);
}

// 0.5*x*(1+erf(x/sqrt2)), unfused as in src/phonon_transformer.c:208-211.
__device__ inline float gelu_erf(float x) {
    const float e = erf_as7126(__fmul_rn(x, 0.7071067811865475244f));
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, e));
}

// gelu_erf with the hardware reciprocal (v_rcp_f32, 1 ulp) and exp2
// (v_exp_f32) in place of the correctly rounded division and libm exp: a
// few ulp from gelu_erf, against the 1.5e-7 error of A&S 7.1.26 itself.
// For the fast prefill, whose activations carry 22 bits.
__device__ inline float gelu_erf_fast(float x) {
    const float z = __fmul_rn(x, 0.7071067811865475244f);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, fabsf(z), 1.0f));
    float r = fmaf(1.061405429f, t, -1.453152027f);
    r = fmaf(r, t, 1.421413741f);
    r = fmaf(r, t, -0.284496736f);
    r = fmaf(r, t, 0.254829592f);
    // e^(-z^2) = 2^(-z^2 log2 e); below 2^-126 it flushes to 0 (erf is 1 there)
    const float neg_exp = -__builtin_amdgcn_exp2f(__fmul_rn(__fmul_rn(z, z), -1.4426950408889634f));
    const float e = copysignf(fmaf(__fmul_rn(t, neg_exp), r, 1.0f), z);
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, e));
}

}  // namespace pgpu
