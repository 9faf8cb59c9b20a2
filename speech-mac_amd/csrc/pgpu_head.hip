// Row kernels of the flow head (src/phonon_sampler.c:229-393) around its
// projections (pgpu_gemm_*): noise scaling, LayerNorm + adaLN modulation into
// split fragments, the time embedding's sincos and RMS scaling, and the
// final Euler update. One wave per 512-wide row where a row is reduced.
#include <cmath>

#include "pgpu_common.hpp"
#include "phonon_gpu.h"

namespace pgpu {
namespace {

// noise = raw * sqrt(T) (src/phonon_sampler.c:371-376) as fp32 rows and as
// split fragments (K = 32) for the input projection. One thread per 8 values.
__global__ __launch_bounds__(256) void k_head_noise(const float *__restrict__ raw, int streams,
                                                    float scale, float *__restrict__ noise,
                                                    uint16_t *__restrict__ xs, int *status) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int s = i >> 2, g = i & 3;
    if (s >= streams) return;
    const float *r = raw + (size_t)s * 32 + g * 8;
    float v[8];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        v[j] = __fmul_rn(r[j], scale);
        bad |= !isfinite(v[j]);
    }
    float *o = noise + (size_t)s * 32 + g * 8;
    *(float4 *)o = make_float4(v[0], v[1], v[2], v[3]);
    *(float4 *)(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    store_split<8>(xs, s, g * 8, 1, v);
    flag_nonfinite(status, bad);
}

// h = LN(x) (eps, optional w and b) then h * (1 + scale) + shift, into split
// fragments (K = 512). Replaces flow_layer_norm and the modulation of
// src/phonon_sampler.c:250-278, 330-334, 350-354: fp32 two-pass moments
// instead of the float cascade mean and double variance; then the same
// element operations in the same order. shift/scale rows: mod + s * ld.
__global__ __launch_bounds__(256) void k_head_ln_mod(const float *__restrict__ x, int streams,
                                                     const float *__restrict__ w,
                                                     const float *__restrict__ b, float eps,
                                                     const float *__restrict__ shift,
                                                     const float *__restrict__ scale, int ld,
                                                     uint16_t *__restrict__ xs, int *status) {
    const int s = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (s >= streams) return;
    const float *row = x + (size_t)s * kWidth + lane * 8;
    const float4 a0 = *(const float4 *)row, a1 = *(const float4 *)(row + 4);
    float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) sum += v[i];
    const float mean = wave_sum(sum) * (1.0f / kWidth);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float c = __fsub_rn(v[i], mean);
        sq = fmaf(c, c, sq);
    }
    const float var = wave_sum(sq) * (1.0f / kWidth);
    const float inverse = 1.0f / sqrtf(__fadd_rn(var, eps));
    const float *sh = shift + (size_t)s * ld + lane * 8, *sc = scale + (size_t)s * ld + lane * 8;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int k = lane * 8 + i;
        float h = __fmul_rn(__fsub_rn(v[i], mean), inverse);
        if (w) h = __fmul_rn(h, w[k]);
        if (b) h = __fadd_rn(h, b[k]);
        const float one_plus_scale = __fadd_rn(1.0f, sc[i]);
        v[i] = __fadd_rn(__fmul_rn(h, one_plus_scale), sh[i]);
        bad |= !isfinite(v[i]);
    }
    store_split<8>(xs, s, lane * 8, kWidth / 32, v);
    flag_nonfinite(status, bad);
}

// [cos | sin](value * freqs[0..128)) as split fragments (K = 256) of
// stream 0 (src/phonon_sampler.c:283-287).
__global__ __launch_bounds__(128) void k_head_time_phase(const float *__restrict__ freqs,
                                                         float value, uint16_t *__restrict__ xs,
                                                         int *status) {
    const int i = threadIdx.x;
    const float phase = __fmul_rn(value, freqs[i]);
    float sn, cs;
    sincosf(phase, &sn, &cs);
    // One value per column: its three terms into the fragment slots.
    uint16_t h, m, l;
    split3(cs, h, m, l);
    const size_t ic = split_index(0, i, 0, 256 / 32);
    xs[ic] = h;
    xs[ic + 512] = m;
    xs[ic + 1024] = l;
    split3(sn, h, m, l);
    const size_t is = split_index(0, 128 + i, 0, 256 / 32);
    xs[is] = h;
    xs[is + 512] = m;
    xs[is + 1024] = l;
    flag_nonfinite(status, !isfinite(cs) || !isfinite(sn));
}

// Both time embeddings' RMS scaling (alpha * out / sqrt(mean(out^2) +
// 1e-5), src/phonon_sampler.c:295-303), then half their sum
// (src/phonon_sampler.c:318-319): tsum = 0.5 * (time_s + time_t). One
// 512-thread work-group: thread i owns column i.
__global__ __launch_bounds__(512) void k_head_time_sum(const float *__restrict__ out0,
                                                       const float *__restrict__ out1,
                                                       const float *__restrict__ alpha0,
                                                       const float *__restrict__ alpha1,
                                                       float *__restrict__ tsum, int *status) {
    __shared__ float part[2][8];
    const int i = threadIdx.x, wave = i >> 6;
    const float a = out0[i], b = out1[i];
    const float sa = wave_sum(__fmul_rn(a, a)), sb = wave_sum(__fmul_rn(b, b));
    if ((i & 63) == 0) {
        part[0][wave] = sa;
        part[1][wave] = sb;
    }
    __syncthreads();
    float ma = 0.0f, mb = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        ma += part[0][w];
        mb += part[1][w];
    }
    const float ia = 1.0f / sqrtf(__fadd_rn(ma * (1.0f / kWidth), 1e-5f));
    const float ib = 1.0f / sqrtf(__fadd_rn(mb * (1.0f / kWidth), 1e-5f));
    const float ts = __fmul_rn(__fmul_rn(alpha0[i], a), ia);
    const float tt = __fmul_rn(__fmul_rn(alpha1[i], b), ib);
    tsum[i] = __fmul_rn(0.5f, __fadd_rn(ts, tt));
    flag_nonfinite(status, !isfinite(tsum[i]));
}

// latent = noise + velocity (src/phonon_sampler.c:380-384); eos[s] =
// eos_rows[s][0] (the one live row of the padded EOS projection).
__global__ __launch_bounds__(256) void k_head_finish(const float *__restrict__ noise,
                                                     const float *__restrict__ velocity,
                                                     int streams, float *__restrict__ latent,
                                                     const float *__restrict__ eos_rows,
                                                     int eos_ld, float *__restrict__ eos,
                                                     int *status) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= streams * 32) return;
    const float y = __fadd_rn(noise[i], velocity[i]);
    latent[i] = y;
    bool bad = !isfinite(y);
    if (eos && (i & 31) == 0) {
        const float e = eos_rows[(size_t)(i >> 5) * eos_ld];
        eos[i >> 5] = e;
        bad |= !isfinite(e);
    }
    flag_nonfinite(status, bad);
}

}  // namespace
}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_head_noise(void *stream, const float *raw, int streams, float temperature,
                               float *noise, uint16_t *noise_split, int *status) {
    if (!raw || streams <= 0 || !noise || !noise_split || !(temperature > 0.0f) ||
        !std::isfinite(temperature))
        return bad_arguments(__func__);
    const float scale = sqrtf(temperature);
    const unsigned blocks = (unsigned)((streams * 4 + 255) / 256);
    hipLaunchKernelGGL(k_head_noise, dim3(blocks), dim3(256), 0, (hipStream_t)stream, raw,
                       streams, scale, noise, noise_split, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_head_ln_mod(void *stream, const float *x, int streams, const float *w,
                                const float *b, float eps, const float *shift, const float *scale,
                                int ld, uint16_t *xs, int *status) {
    if (!x || streams <= 0 || !shift || !scale || ld < kWidth || ld % 4 || !xs)
        return bad_arguments(__func__);
    hipLaunchKernelGGL(k_head_ln_mod, dim3((unsigned)((streams + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, x, streams, w, b, eps, shift, scale, ld, xs, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_head_time_phase(void *stream, const float *freqs, float value, uint16_t *xs,
                                    int *status) {
    if (!freqs || !xs || !std::isfinite(value)) return bad_arguments(__func__);
    hipLaunchKernelGGL(k_head_time_phase, dim3(1), dim3(128), 0, (hipStream_t)stream, freqs,
                       value, xs, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_head_time_sum(void *stream, const float *out0, const float *out1,
                                  const float *alpha0, const float *alpha1, float *tsum,
                                  int *status) {
    if (!out0 || !out1 || !alpha0 || !alpha1 || !tsum) return bad_arguments(__func__);
    hipLaunchKernelGGL(k_head_time_sum, dim3(1), dim3(512), 0, (hipStream_t)stream, out0, out1,
                       alpha0, alpha1, tsum, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_head_finish(void *stream, const float *noise, const float *velocity,
                                int streams, float *latent, const float *eos_rows, int eos_ld,
                                float *eos, int *status) {
    if (!noise || !velocity || streams <= 0 || !latent || (eos && (!eos_rows || eos_ld < 1)))
        return bad_arguments(__func__);
    const unsigned blocks = (unsigned)((streams * 32 + 255) / 256);
    hipLaunchKernelGGL(k_head_finish, dim3(blocks), dim3(256), 0, (hipStream_t)stream, noise,
                       velocity, streams, latent, eos_rows, eos_ld, eos, status);
    return launch_ok(__func__);
}
