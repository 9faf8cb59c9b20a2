// Launches of the flow head (src/phonon_sampler.c:229-393): its projections
// (the tasks of pgpu_gemm.hpp, BF16 weights) grouped so that one launch runs
// every projection whose inputs are ready, with the row work fused into
// them: noise scaling beside the first projections, LayerNorm + adaLN
// modulation in front of each block's first MLP projection and of the final
// layer, the Euler update and the EOS copy in the final launch. A step of B
// streams is 15 launches: front, modulation + input, 6 x (MLP in, MLP out),
// final. The fused chain (pgpu_head_block) makes each block one launch:
// the block's MLP-in work-groups also multiply their 64 hidden columns by
// the MLP-out matrix, and the next launch adds the 8 partials in the
// MLP-out projection's own order (9 launches, the same bits). The time
// embedding's sincos and RMS scaling run once per (s, t).
#include <cmath>

#include "pgpu_gemm.hpp"
#include "phonon_gpu.h"

namespace pgpu {
namespace {

// noise = raw * scale (src/phonon_sampler.c:371-376 with scale = sqrt(T))
// as fp32 rows and as split fragments (K = 32) for the input projection.
// One thread per 8 values; `first` is the thread index of this block's
// thread 0.
__device__ inline void noise_rows(const float *__restrict__ raw, int streams, float scale,
                                  float *__restrict__ noise, uint16_t *__restrict__ xs,
                                  int *status, int first) {
    const int i = first + threadIdx.x;
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

// One projection task of a launch that runs several projections: `index`
// counts the projection's own work-groups (row group fastest, then the
// 16-stream tile).
template <int SRC, int EPI>
__device__ inline void wide_at(const GemmArgs &a, int index, uint16_t *lds) {
    const int groups = (a.n_rows / 16 + 3) / 4;
    gemm_wide_task<SRC, EPI, false>(a, index % groups, index / groups, lds, NoWait{});
}

template <int EPI>
__device__ inline void split_at(const GemmArgs &a, int index, uint16_t *lds) {
    const int tiles = a.n_rows / 16;
    gemm_split_task<EPI, false>(a, index % tiles, index / tiles, lds, NoWait{});
}

__host__ __device__ inline int wide_groups(const GemmArgs &a) {
    return (a.n_rows / 16 + 3) / 4 * ((a.streams + 15) / 16);
}

__host__ __device__ inline int split_groups(const GemmArgs &a) {
    return a.n_rows / 16 * ((a.streams + 15) / 16);
}

struct NoiseArgs {
    const float *raw;
    float scale;
    float *noise;
    uint16_t *xs;
};

// First launch of a head step: the condition's projection into split
// fragments of SiLU(y) (y = cond_embed(c) + tsum), the EOS row of the
// condition (optional) and the noise rows; none depends on another. With
// SRC = SRC_LN the condition is the LayerNorm of the rows (the decoder's
// output norm), computed in both projections' prologues.
template <int SRC>
__global__ __launch_bounds__(kTaskThreads) void k_head_front(GemmArgs cond, GemmArgs eos,
                                                             int with_eos, NoiseArgs nz) {
    __shared__ uint4 lds4[kTaskLds / 8];
    uint16_t *lds = (uint16_t *)lds4;
    int b = blockIdx.x;
    const int n_cond = wide_groups(cond);
    if (b < n_cond) return wide_at<SRC, EPI_SILU_SPLIT>(cond, b, lds);
    b -= n_cond;
    if (with_eos) {
        if (b < wide_groups(eos)) return wide_at<SRC, EPI_STORE>(eos, b, lds);
        b -= wide_groups(eos);
    }
    noise_rows(nz.raw, cond.streams, nz.scale, nz.noise, nz.xs, cond.status, b * kTaskThreads);
}

// Second launch: the seven adaLN projections as one (reading SiLU(y); each
// work-group copies its 16 streams' fragments into LDS once for 64 rows) and
// the input projection of the noise.
__global__ __launch_bounds__(kTaskThreads) void k_head_mod(GemmArgs ada, GemmArgs input) {
    __shared__ uint4 lds4[kTaskLds / 8];
    uint16_t *lds = (uint16_t *)lds4;
    const int b = blockIdx.x, n_ada = wide_groups(ada);
    if (b < n_ada) return wide_at<SRC_SPLIT_LDS, EPI_STORE>(ada, b, lds);
    split_at<EPI_STORE>(input, b - n_ada, lds);
}

// A block's first MLP projection with its LayerNorm and modulation fused in
// front: split fragments of SiLU(mlp_0(LN(x) * (1 + scale) + shift)).
__global__ __launch_bounds__(kTaskThreads) void k_head_mlp_in(GemmArgs a) {
    __shared__ uint4 lds4[kTaskLds / 8];
    wide_at<SRC_LN_MOD, EPI_SILU_SPLIT>(a, blockIdx.x, (uint16_t *)lds4);
}

// A residual block of the fused chain, one launch: x (the rows, SRC_LN_MOD,
// or the previous block's output from its partials, SRC_LN_MOD_PARTS, each
// work-group storing its 64 dimensions of it), LayerNorm + modulation, the
// MLP-in projection + SiLU of the work-group's 64 hidden columns, and their
// product with the MLP-out matrix: partial bx of the block
// ([ld_parts][512] at parts_out + bx * ld_parts * 512).
template <int SRC>
__global__ __launch_bounds__(kTaskThreads) void k_head_block(GemmArgs a, int ld_parts) {
    __shared__ uint4 lds4[kTaskLds / 8];
    constexpr int groups = kWidth / 64;
    const int bx = (int)blockIdx.x % groups, st = (int)blockIdx.x / groups;
    a.tmlp_out += (size_t)bx * ld_parts * kWidth;
    a.pub0 = bx * 64;
    gemm_wide_task<SRC, EPI_SILU_W2, false>(a, bx, st, (uint16_t *)lds4, NoWait{});
}

// Last launch: the final layer on the modulated LayerNorm of x (SRC_LN_MOD:
// the rows; SRC_LN_MOD_PARTS: the last block's output from its partials),
// either the velocity (EPI_STORE) or noise + velocity (EPI_GATED with a gate
// of ones, exact); one more work-group copies the EOS logits out of their
// padded rows.
template <int SRC, int EPI>
__global__ __launch_bounds__(kTaskThreads) void k_head_final(GemmArgs a, const float *eos_rows,
                                                             int eos_ld, float *eos) {
    __shared__ uint4 lds4[kTaskLds / 8];
    const int n = wide_groups(a);
    if ((int)blockIdx.x < n) return wide_at<SRC, EPI>(a, blockIdx.x, (uint16_t *)lds4);
    bool bad = false;
    for (int s = threadIdx.x; s < a.streams; s += kTaskThreads) {
        const float e = eos_rows[(size_t)s * eos_ld];
        eos[s] = e;
        bad |= !isfinite(e);
    }
    flag_nonfinite(a.status, bad);
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

}  // namespace
}  // namespace pgpu

using namespace pgpu;

static bool bf16_matrix(const pgpu_matrix *w, size_t rows, size_t columns) {
    return w && w->values && !w->q8 && w->rows == rows && w->columns == columns;
}

static GemmArgs head_args(const pgpu_matrix *w, int streams, int *status) {
    GemmArgs a{};
    a.w = w->values;
    a.n_rows = (int)w->rows;
    a.k_cols = (int)w->columns;
    a.streams = streams;
    a.status = status;
    return a;
}

extern "C" int pgpu_head_front(void *stream, const pgpu_matrix *cond_w, const float *conditions,
                               int streams, const float *norm_w, const float *norm_b,
                               const float *cond_bias, const float *tsum,
                               uint16_t *silu_split, const pgpu_matrix *eos_w,
                               const float *eos_bias, float *eos_rows, int eos_ld,
                               const float *raw, float scale, float *noise,
                               uint16_t *noise_split, int *status) {
    if (!bf16_matrix(cond_w, kWidth, kWidth) || !conditions || streams <= 0 || !silu_split ||
        (!norm_w) != (!norm_b) ||
        !raw || !noise || !noise_split || !(scale > 0.0f) || !std::isfinite(scale) ||
        (eos_w && (!bf16_matrix(eos_w, 16, kWidth) || !eos_rows || eos_ld < 16 || eos_ld % 4)))
        return bad_arguments(__func__);
    GemmArgs cond = head_args(cond_w, streams, status);
    cond.ln_x = conditions;
    cond.ln_w = norm_w;
    cond.ln_b = norm_b;
    cond.ln_eps = 1e-5f;
    cond.bias = cond_bias;
    cond.bias2 = tsum;
    cond.out_split = silu_split;
    cond.out_kb = kWidth / 32;
    GemmArgs eos{};
    if (eos_w) {
        eos = head_args(eos_w, streams, status);
        eos.ln_x = conditions;
        eos.ln_w = norm_w;
        eos.ln_b = norm_b;
        eos.ln_eps = 1e-5f;
        eos.bias = eos_bias;
        eos.out = eos_rows;
        eos.ld_out = eos_ld;
    }
    const NoiseArgs nz{raw, scale, noise, noise_split};
    const int blocks = wide_groups(cond) + (eos_w ? wide_groups(eos) : 0) +
                       (streams * 4 + kTaskThreads - 1) / kTaskThreads;
    if (norm_w)
        hipLaunchKernelGGL(k_head_front<SRC_LN>, dim3((unsigned)blocks), dim3(kTaskThreads), 0,
                           (hipStream_t)stream, cond, eos, eos_w != nullptr, nz);
    else
        hipLaunchKernelGGL(k_head_front<SRC_ROWS>, dim3((unsigned)blocks), dim3(kTaskThreads),
                           0, (hipStream_t)stream, cond, eos, eos_w != nullptr, nz);
    return launch_ok(__func__);
}

extern "C" int pgpu_head_mod(void *stream, const pgpu_matrix *ada_w, const uint16_t *silu_split,
                             int streams, const float *ada_bias, float *mod, int ld_mod,
                             const pgpu_matrix *input_w, const uint16_t *noise_split,
                             const float *input_bias, float *x, int *status) {
    if (!ada_w || !bf16_matrix(ada_w, ada_w->rows, kWidth) || ada_w->rows % 16 || !silu_split ||
        streams <= 0 || !mod || ld_mod < (int)ada_w->rows || ld_mod % 4 ||
        !bf16_matrix(input_w, kWidth, 32) || !noise_split || !x)
        return bad_arguments(__func__);
    GemmArgs ada = head_args(ada_w, streams, status);
    ada.xs = silu_split;
    ada.bias = ada_bias;
    ada.out = mod;
    ada.ld_out = ld_mod;
    GemmArgs input = head_args(input_w, streams, status);
    input.xs = noise_split;
    input.bias = input_bias;
    input.out = x;
    input.ld_out = kWidth;
    const int blocks = wide_groups(ada) + split_groups(input);
    hipLaunchKernelGGL(k_head_mod, dim3((unsigned)blocks), dim3(kTaskThreads), 0,
                       (hipStream_t)stream, ada, input);
    return launch_ok(__func__);
}

extern "C" int pgpu_head_mlp_in(void *stream, const pgpu_matrix *w, const float *x, int streams,
                                const float *norm_w, const float *norm_b, float eps,
                                const float *mod, int ld_mod, const float *bias,
                                uint16_t *out_split, int *status) {
    if (!bf16_matrix(w, kWidth, kWidth) || !x || streams <= 0 || !mod || ld_mod < 2 * kWidth ||
        ld_mod % 4 || !out_split || !(eps > 0.0f))
        return bad_arguments(__func__);
    GemmArgs a = head_args(w, streams, status);
    a.ln_x = x;
    a.ln_w = norm_w;
    a.ln_b = norm_b;
    a.ln_eps = eps;
    a.mod = mod;
    a.ld_mod = ld_mod;
    a.bias = bias;
    a.out_split = out_split;
    a.out_kb = kWidth / 32;
    hipLaunchKernelGGL(k_head_mlp_in, dim3((unsigned)wide_groups(a)), dim3(kTaskThreads), 0,
                       (hipStream_t)stream, a);
    return launch_ok(__func__);
}

// The previous block's partials (pgpu_head_parts) checked and set into a.
static bool set_parts(GemmArgs &a, const pgpu_head_parts *prev, int streams) {
    if (!prev->parts || prev->ld_parts < streams || !prev->gate || prev->ld_gate < kWidth ||
        prev->ld_gate % 4 || prev->ld_parts % 4)
        return false;
    a.tmlp = prev->parts;
    a.mlp_streams = prev->ld_parts;
    a.part_gate = prev->gate;
    a.ld_part_gate = prev->ld_gate;
    a.part_bias = prev->bias;
    return true;
}

// True if [a, a + na) and [b, b + nb) (floats) share an address.
static bool overlap(const float *a, size_t na, const float *b, size_t nb) {
    return a < b + nb && b < a + na;
}

extern "C" int pgpu_head_block(void *stream, const pgpu_matrix *w_in, const pgpu_matrix *w_out,
                               const float *x, int streams, const pgpu_head_parts *prev,
                               float *x_out, const float *norm_w, const float *norm_b, float eps,
                               const float *mod, int ld_mod, const float *in_bias,
                               float *parts_out, int ld_parts, int *status) {
    if (!bf16_matrix(w_in, kWidth, kWidth) || !bf16_matrix(w_out, kWidth, kWidth) || !x ||
        streams <= 0 || !mod || ld_mod < 2 * kWidth || ld_mod % 4 || !(eps > 0.0f) ||
        !parts_out || ld_parts < streams || ld_parts % 4 || (prev && !x_out))
        return bad_arguments(__func__);
    const size_t rows = (size_t)streams * kWidth, parts = (size_t)8 * ld_parts * kWidth;
    GemmArgs a = head_args(w_in, streams, status);
    if (prev) {
        if (!set_parts(a, prev, streams) || overlap(x_out, rows, x, rows) ||
            overlap(parts_out, parts, prev->parts, (size_t)8 * prev->ld_parts * kWidth) ||
            overlap(x_out, rows, parts_out, parts))
            return bad_arguments(__func__);
        a.x_pub = x_out;
    }
    a.ln_x = x;
    a.ln_w = norm_w;
    a.ln_b = norm_b;
    a.ln_eps = eps;
    a.mod = mod;
    a.ld_mod = ld_mod;
    a.bias = in_bias;
    a.w2 = w_out->values;
    a.tmlp_out = parts_out;
    const dim3 grid((unsigned)wide_groups(a)), block(kTaskThreads);
    if (prev)
        hipLaunchKernelGGL(k_head_block<SRC_LN_MOD_PARTS>, grid, block, 0, (hipStream_t)stream, a,
                           ld_parts);
    else
        hipLaunchKernelGGL(k_head_block<SRC_LN_MOD>, grid, block, 0, (hipStream_t)stream, a,
                           ld_parts);
    return launch_ok(__func__);
}

extern "C" int pgpu_head_final(void *stream, const pgpu_matrix *w, const float *x, int streams,
                               const pgpu_head_parts *prev, float eps, const float *mod,
                               int ld_mod, const float *bias, const float *residual,
                               const float *ones, float *out, uint16_t *out_split,
                               const float *eos_rows, int eos_ld, float *eos, int *status) {
    if (!w || !bf16_matrix(w, w->rows, kWidth) || w->rows % 16 || !x || streams <= 0 || !mod ||
        ld_mod < 2 * kWidth || ld_mod % 4 || !out || (residual && !ones) || !(eps > 0.0f) ||
        (eos && (!eos_rows || eos_ld < 1)) || (out_split && (!residual || w->rows % 32)))
        return bad_arguments(__func__);
    GemmArgs a = head_args(w, streams, status);
    if (prev && !set_parts(a, prev, streams))
        return bad_arguments(__func__);
    a.ln_x = x;
    a.ln_eps = eps;
    // With a residual: the output's split fragments too, w->rows / 32 column
    // blocks per row (whole 32-column blocks only).
    a.out_split = out_split;
    a.out_kb = (int)w->rows / 32;
    a.mod = mod;
    a.ld_mod = ld_mod;
    a.bias = bias;
    a.out = out;
    a.ld_out = (int)w->rows;
    const unsigned blocks = (unsigned)wide_groups(a) + (eos ? 1u : 0u);
    if (residual) {
        a.residual = residual;
        a.gate = ones;
        a.ld_gate = 0;
    }
    const hipStream_t st = (hipStream_t)stream;
    if (residual && prev)
        hipLaunchKernelGGL((k_head_final<SRC_LN_MOD_PARTS, EPI_GATED>), dim3(blocks),
                           dim3(kTaskThreads), 0, st, a, eos_rows, eos_ld, eos);
    else if (residual)
        hipLaunchKernelGGL((k_head_final<SRC_LN_MOD, EPI_GATED>), dim3(blocks), dim3(kTaskThreads),
                           0, st, a, eos_rows, eos_ld, eos);
    else if (prev)
        hipLaunchKernelGGL((k_head_final<SRC_LN_MOD_PARTS, EPI_STORE>), dim3(blocks),
                           dim3(kTaskThreads), 0, st, a, eos_rows, eos_ld, eos);
    else
        hipLaunchKernelGGL((k_head_final<SRC_LN_MOD, EPI_STORE>), dim3(blocks), dim3(kTaskThreads),
                           0, st, a, eos_rows, eos_ld, eos);
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

// ---------------------------------------------------------------------------
// The LSD step as one launch (pgpu_head_flow in phonon_gpu.h): the tasks of
// the launches above, each first waiting for per-tile counters.
namespace pgpu {
namespace {

constexpr uint64_t kHeadWaitTicks = 100000000ull;  // 1 s at 100 MHz

__device__ inline unsigned *head_counter(const pgpu_head_flow &f, int tile, int which) {
    return f.counters + ((size_t)tile * PGPU_HEADC_KINDS + which) * PGPU_HEAD_COUNTER_STRIDE;
}

// Up to three (counter, target) conditions (unused: null counter): one lane
// polls them in turn (each poll loads the counter and the status word
// together), then the work-group barrier releases the task. A wait that
// exceeds `ticks` of the 100 MHz clock, or sees another task's give-up,
// sets status value 4 and stops waiting, so the launch always ends.
struct HeadWait {
    const unsigned *flag0, *flag1, *flag2;
    unsigned target0, target1, target2;
    int *status;
    uint64_t ticks;
    __device__ bool poll(const unsigned *flag, unsigned target, uint64_t t0) const {
        for (;;) {
            const unsigned count =
                __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int st = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (count >= target) return true;
            if ((st & 4) || wall_clock64() - t0 > ticks) {
                atomicOr(status, 4);
                return false;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __device__ void operator()() const {
        if (threadIdx.x == 0) {
            const uint64_t t0 = wall_clock64();
            bool ok = !flag0 || poll(flag0, target0, t0);
            ok = ok && (!flag1 || poll(flag1, target1, t0));
            ok = ok && (!flag2 || poll(flag2, target2, t0));
        }
        __syncthreads();
    }
};

// The wait for (which, target) pairs of this tile's counters (which < 0:
// none).
__device__ inline HeadWait head_wait(const pgpu_head_flow &f, int tile, int c0 = -1,
                                     unsigned t0 = 0, int c1 = -1, unsigned t1 = 0,
                                     int c2 = -1, unsigned t2 = 0) {
    HeadWait w;
    w.flag0 = c0 < 0 ? nullptr : head_counter(f, tile, c0);
    w.flag1 = c1 < 0 ? nullptr : head_counter(f, tile, c1);
    w.flag2 = c2 < 0 ? nullptr : head_counter(f, tile, c2);
    w.target0 = t0;
    w.target1 = t1;
    w.target2 = t2;
    w.status = f.status;
    w.ticks = f.wait_us ? (uint64_t)f.wait_us * 100u : kHeadWaitTicks;
    return w;
}

// Completes a task: every wave's write-through stores have drained, then
// one lane counts it.
__device__ inline void head_signal(const pgpu_head_flow &f, int tile, int which) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(head_counter(f, tile, which), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline GemmArgs flow_args(const pgpu_head_flow &f, const pgpu_matrix &w) {
    GemmArgs a{};
    a.w = w.values;
    a.n_rows = (int)w.rows;
    a.k_cols = (int)w.columns;
    a.streams = f.streams;
    a.status = f.status;
    a.wt_out = true;  // read by tasks on other XCDs within the launch
    return a;
}

__device__ inline float *x_rows(const pgpu_head_flow &f, int version) {
    return f.x + (size_t)version * f.tiles * 16 * kWidth;
}

__device__ inline uint16_t *u_rows(const pgpu_head_flow &f, int block) {
    return f.u_split + (size_t)block * f.tiles * (kWidth / 32) * 1536;
}

// Tagged hand-off rows: x version v, SiLU(u) of block b ([tiles*16][512]).
__device__ inline uint64_t *tx_rows(const pgpu_head_flow &f, int version) {
    return f.tx + (size_t)version * f.tiles * 16 * kWidth;
}

__device__ inline uint64_t *tu_rows(const pgpu_head_flow &f, int block) {
    return f.tu + (size_t)block * f.tiles * 16 * kWidth;
}

constexpr int kAdaRows = 3 * kWidth;                 // one block's shift, scale, gate
constexpr int kModCols = PGPU_HEAD_BLOCKS * kAdaRows + 2 * kWidth;
constexpr int kAdaGroupsPerBlock = kAdaRows / 64;    // 24
constexpr int kFinalAdaGroups = 2 * kWidth / 64;     // 16

__global__ __launch_bounds__(kTaskThreads) void k_head_flow(pgpu_head_flow f) {
    __shared__ uint4 lds4[kTaskLds / 8];
    uint16_t *lds = (uint16_t *)lds4;
    const uint32_t d = f.schedule[blockIdx.x];
    const int kind = d & 15, blk = (d >> 4) & 15, tile = (d >> 8) & 255, index = (int)(d >> 16);
    // Tagged mode: x and u go from task to task as tagged words, polled by
    // their consumers (the other hand-offs keep their counters).
    const bool tagged = f.tagged != 0;
    const TagPoll tp{tagged ? __hip_atomic_load(f.tag_word, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0u,
                     f.status, f.wait_us ? (uint64_t)f.wait_us * 100u : kHeadWaitTicks, false};
    switch (kind) {
    case PGPU_HEAD_COND: {
        GemmArgs a = flow_args(f, f.cond_w);
        a.ln_x = f.conditions;
        a.ln_w = f.out_norm;
        a.ln_b = f.out_norm ? f.out_norm + kWidth : nullptr;
        a.ln_eps = 1e-5f;
        a.bias = f.b_cond;
        a.bias2 = f.tsum;
        a.out_split = f.silu_split;
        a.out_kb = kWidth / 32;
        if (f.out_norm)
            gemm_wide_task<SRC_LN, EPI_SILU_SPLIT, false>(a, index, tile, lds, NoWait{});
        else
            gemm_wide_task<SRC_ROWS, EPI_SILU_SPLIT, false>(a, index, tile, lds, NoWait{});
        head_signal(f, tile, PGPU_HEADC_COND);
        break;
    }
    case PGPU_HEAD_EOS: {
        GemmArgs a = flow_args(f, f.eos_w);
        a.ln_x = f.conditions;
        a.ln_w = f.out_norm;
        a.ln_b = f.out_norm ? f.out_norm + kWidth : nullptr;
        a.ln_eps = 1e-5f;
        a.bias = f.b_eos;
        a.out = f.eos_rows;
        a.ld_out = 16;
        if (f.out_norm)
            gemm_wide_task<SRC_LN, EPI_STORE, false>(a, 0, tile, lds, NoWait{});
        else
            gemm_wide_task<SRC_ROWS, EPI_STORE, false>(a, 0, tile, lds, NoWait{});
        head_signal(f, tile, PGPU_HEADC_EOS);
        break;
    }
    case PGPU_HEAD_NOISE: {
        // noise = raw * scale (src/phonon_sampler.c:371-376), 8 values per
        // thread: rows and split fragments, both written through.
        const int i = threadIdx.x, s = tile * 16 + (i >> 2), g = i & 3;
        if (i < 64 && s < f.streams) {
            const float *r = f.raw + (size_t)s * 32 + g * 8;
            float v[8];
            bool bad = false;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                v[j] = __fmul_rn(r[j], f.scale);
                bad |= !isfinite(v[j]);
            }
            float *o = f.noise + (size_t)s * 32 + g * 8;
            store_wt(o, make_float4(v[0], v[1], v[2], v[3]));
            store_wt(o + 4, make_float4(v[4], v[5], v[6], v[7]));
            store_split4(f.noise_split, s, g * 8, 1, v, true);
            store_split4(f.noise_split, s, g * 8 + 4, 1, v + 4, true);
            flag_nonfinite(f.status, bad);
        }
        head_signal(f, tile, PGPU_HEADC_NOISE);
        break;
    }
    case PGPU_HEAD_INPUT: {
        GemmArgs a = flow_args(f, f.input_w);
        a.xs = f.noise_split;
        a.bias = f.b_input;
        a.out = x_rows(f, 0);
        a.ld_out = kWidth;
        if (tagged) a.tout = tx_rows(f, 0), a.tp = tp;
        gemm_split_task<EPI_STORE, false>(a, index, tile, lds,
                                          head_wait(f, tile, PGPU_HEADC_NOISE, 1u));
        if (!tagged) head_signal(f, tile, PGPU_HEADC_X);
        break;
    }
    case PGPU_HEAD_ADA: {
        GemmArgs a = flow_args(f, f.ada_w);
        a.xs = f.silu_split;
        a.bias = f.b_ada;
        a.out = f.mod;
        a.ld_out = kModCols;
        gemm_wide_task<SRC_SPLIT_LDS, EPI_STORE, false>(
            a, index, tile, lds, head_wait(f, tile, PGPU_HEADC_COND, (kWidth / 16 + 3) / 4));
        head_signal(f, tile, PGPU_HEADC_ADA + index / kAdaGroupsPerBlock);
        break;
    }
    case PGPU_HEAD_MLP_IN: {
        GemmArgs a = flow_args(f, f.mlp_w[blk][0]);
        a.ln_x = x_rows(f, blk);
        a.ln_w = f.norm_w[blk];
        a.ln_b = f.norm_b[blk];
        a.ln_eps = 1e-6f;
        a.mod = f.mod + (size_t)blk * kAdaRows;
        a.ld_mod = kModCols;
        a.bias = f.b_mlp[blk][0];
        a.out_split = u_rows(f, blk);
        a.out_kb = kWidth / 32;
        if (tagged) {
            a.tx = tx_rows(f, blk);
            a.tout = tu_rows(f, blk);
            a.tp = tp;
            gemm_wide_task<SRC_LN_MOD, EPI_SILU_SPLIT, false>(
                a, index, tile, lds,
                head_wait(f, tile, PGPU_HEADC_ADA + blk, kAdaGroupsPerBlock));
            break;
        }
        gemm_wide_task<SRC_LN_MOD, EPI_SILU_SPLIT, false>(
            a, index, tile, lds,
            head_wait(f, tile, PGPU_HEADC_X + blk, kWidth / 16, PGPU_HEADC_ADA + blk,
                      kAdaGroupsPerBlock));
        head_signal(f, tile, PGPU_HEADC_U + blk);
        break;
    }
    case PGPU_HEAD_MLP_OUT: {
        GemmArgs a = flow_args(f, f.mlp_w[blk][1]);
        a.xs = u_rows(f, blk);
        a.bias = f.b_mlp[blk][1];
        a.gate = f.mod + (size_t)blk * kAdaRows + 2 * kWidth;
        a.ld_gate = kModCols;
        a.residual = x_rows(f, blk);
        a.out = x_rows(f, blk + 1);
        a.ld_out = kWidth;
        if (tagged) {
            a.tx = tu_rows(f, blk);
            a.tres = tx_rows(f, blk);
            a.tout = tx_rows(f, blk + 1);
            a.tp = tp;
            // The gate rows come from the block's ADA tasks: nothing the task
            // polls implies they are done (the counted chain's MLP_IN count
            // did), so their count is waited for.
            gemm_split_task<EPI_GATED, false>(
                a, index, tile, lds, head_wait(f, tile, PGPU_HEADC_ADA + blk, kAdaGroupsPerBlock));
            break;
        }
        gemm_split_task<EPI_GATED, false>(a, index, tile, lds,
                                          head_wait(f, tile, PGPU_HEADC_U + blk,
                                                    (kWidth / 16 + 3) / 4));
        head_signal(f, tile, PGPU_HEADC_X + blk + 1);
        break;
    }
    case PGPU_HEAD_FINAL: {
        GemmArgs a = flow_args(f, f.final_w);
        a.ln_x = x_rows(f, PGPU_HEAD_BLOCKS);
        a.ln_eps = 1e-6f;
        a.out_split = f.latent_split;
        a.out_kb = (int)f.final_w.rows / 32;
        a.mod = f.mod + (size_t)PGPU_HEAD_BLOCKS * kAdaRows;
        a.ld_mod = kModCols;
        a.bias = f.b_final;
        a.out = f.latents;
        a.ld_out = (int)f.final_w.rows;
        a.residual = f.noise;
        a.gate = f.ones;
        a.ld_gate = 0;
        if (tagged) {
            a.tx = tx_rows(f, PGPU_HEAD_BLOCKS);
            a.tp = tp;
        }
        gemm_wide_task<SRC_LN_MOD, EPI_GATED, false>(
            a, 0, tile, lds,
            tagged ? head_wait(f, tile, PGPU_HEADC_ADA + PGPU_HEAD_BLOCKS, kFinalAdaGroups,
                               f.with_eos ? PGPU_HEADC_EOS : -1, 1u)
                   : head_wait(f, tile, PGPU_HEADC_X + PGPU_HEAD_BLOCKS, kWidth / 16,
                               PGPU_HEADC_ADA + PGPU_HEAD_BLOCKS, kFinalAdaGroups,
                               f.with_eos ? PGPU_HEADC_EOS : -1, 1u));
        if (f.with_eos && f.eos) {
            const int s = tile * 16 + (int)threadIdx.x;
            if (threadIdx.x < 16 && s < f.streams) {
                const float e = f.eos_rows[(size_t)s * 16];
                f.eos[s] = e;
                flag_nonfinite(f.status, !isfinite(e));
            }
        }
        head_signal(f, tile, PGPU_HEADC_FINAL);
        break;
    }
    case PGPU_HEAD_EMBED: {
        GemmArgs a = flow_args(f, f.embed_w);
        a.xs = f.latent_split;
        a.out = f.next;
        a.ld_out = kWidth;
        a.residual = f.embed_in;
        a.wt_out = false;  // read after the launch only
        gemm_split_task<EPI_RESIDUAL, false>(a, index, tile, lds,
                                             head_wait(f, tile, PGPU_HEADC_FINAL, 1u));
        break;
    }
    default:
        break;
    }
}

__global__ void k_head_flow_reset(unsigned *counters, size_t n, unsigned *tag_word) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        counters[i] = 0u;
    if (tag_word && blockIdx.x == 0 && threadIdx.x == 0) *tag_word = *tag_word + 1u;
}

}  // namespace
}  // namespace pgpu

extern "C" int pgpu_head_flow_launch(void *stream, const pgpu_head_flow *f) {
    if (!f || !f->schedule || f->tasks <= 0 || f->streams <= 0 ||
        f->tiles != (f->streams + 15) / 16 || f->tiles > 255 ||
        !bf16_matrix(&f->cond_w, kWidth, kWidth) || !bf16_matrix(&f->input_w, kWidth, 32) ||
        !bf16_matrix(&f->ada_w, (size_t)pgpu::kModCols, kWidth) ||
        !bf16_matrix(&f->final_w, 32, kWidth) || !f->conditions || !f->b_cond || !f->tsum ||
        !f->b_ada || !f->b_input || !f->b_final || !f->raw || !(f->scale > 0.0f) ||
        !std::isfinite(f->scale) || !f->noise || !f->noise_split || !f->silu_split || !f->mod ||
        !f->x || !f->u_split || !f->ones || !f->latents || !f->counters || !f->status ||
        (f->with_eos && (!bf16_matrix(&f->eos_w, 16, kWidth) || !f->eos_rows)) ||
        (f->with_embed && (!bf16_matrix(&f->embed_w, kWidth, 32) || !f->latent_split ||
                           !f->embed_in || !f->next)) ||
        (f->tagged && (!f->tx || !f->tu || !f->tag_word)))
        return bad_arguments("pgpu_head_flow_launch");
    for (int b = 0; b < PGPU_HEAD_BLOCKS; b++)
        if (!bf16_matrix(&f->mlp_w[b][0], kWidth, kWidth) ||
            !bf16_matrix(&f->mlp_w[b][1], kWidth, kWidth) || !f->norm_w[b] || !f->norm_b[b])
            return bad_arguments("pgpu_head_flow_launch");
    hipLaunchKernelGGL(pgpu::k_head_flow, dim3((unsigned)f->tasks), dim3(kTaskThreads), 0,
                       (hipStream_t)stream, *f);
    return launch_ok("pgpu_head_flow_launch");
}

extern "C" int pgpu_head_flow_reset(void *stream, unsigned *counters, size_t count,
                                    unsigned *tag_word) {
    if (!counters || !count) return bad_arguments("pgpu_head_flow_reset");
    const unsigned blocks = (unsigned)((count + 255) / 256 < 64 ? (count + 255) / 256 : 64);
    hipLaunchKernelGGL(pgpu::k_head_flow_reset, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       counters, count, tag_word);
    return launch_ok("pgpu_head_flow_reset");
}
