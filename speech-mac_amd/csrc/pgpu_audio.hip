// Audio decoder kernels: the Mimi latent transformer's own steps
// (src/phonon_mimi.c) and the SEANet convolutions (src/phonon_conv.c). The
// Mimi projections run on the MFMA projection kernels (pgpu_gemm.hip).
//
// Every kernel works on all positions of a request at once: a causal
// convolution's output position t reads the input window it needs, taking
// the positions before the call from the state's history; a transposed
// convolution's position t recomputes the overlap of position t - 1 (the
// same dot product the sequential form carries over). Positions are rows of
// a row-major [positions][channels] array.
//
// Dot products run over input channels, then taps, as a sequential fp32
// sum with separate multiply and add (the sequential form of the
// reference's BLAS calls), one thread per output channel: the weights are
// stored [input channel][tap][output channel] so that a wave's loads are
// contiguous.
#include "pgpu_common.hpp"
#include "phonon_gpu.h"

namespace pgpu {
namespace {

constexpr int kMimiRows = 16;  // feature rows per latent frame

// Projection (512 x 32) and depthwise upsample of every latent frame:
// hidden[16 f + o][c] = prev[c] * k[c][16 + o] + cur[c] * k[c][o], where
// cur is frame f's projection and prev frame f - 1's (the state's
// `previous` for f = 0). The last frame's projection becomes `previous`.
__global__ __launch_bounds__(256) void k_mimi_input(const float *__restrict__ latents, int frames,
                                                    const float *__restrict__ proj,
                                                    const float *__restrict__ upk,
                                                    float *__restrict__ previous,
                                                    float *__restrict__ hidden, int *status) {
    const int f = blockIdx.x, c = blockIdx.y * 256 + threadIdx.x;
    auto project = [&](int frame) {
        float dot = 0.0f;
#pragma unroll 8
        for (int i = 0; i < 32; i++) dot = dot + proj[c * 32 + i] * latents[frame * 32 + i];
        return dot;
    };
    const float cur = project(f);
    const float prev = f == 0 ? previous[c] : project(f - 1);
    bool bad = !isfinite(cur) || !isfinite(prev);
#pragma unroll
    for (int o = 0; o < kMimiRows; o++) {
        const float current = cur * upk[c * 32 + o];
        const float old = prev * upk[c * 32 + kMimiRows + o];
        const float v = old + current;
        bad |= !isfinite(v);
        hidden[((size_t)f * kMimiRows + o) * kWidth + c] = v;
    }
    flag_nonfinite(status, bad);
    // Every block reads `previous` (f = 0 only) before any block writes it:
    // the write is done by a separate launch (k_mimi_keep_previous).
}

__global__ void k_mimi_keep_previous(const float *__restrict__ latents, int frame,
                                     const float *__restrict__ proj, float *__restrict__ previous) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    float dot = 0.0f;
#pragma unroll 8
    for (int i = 0; i < 32; i++) dot = dot + proj[c * 32 + i] * latents[frame * 32 + i];
    previous[c] = dot;
}

// RoPE of q and k of every row (position first + r), then k and v into the
// ring slot of that position.
__global__ __launch_bounds__(256) void k_mimi_rope_store(float *__restrict__ qkv, int rows,
                                                         long long first,
                                                         const float2 *__restrict__ rope,
                                                         float *__restrict__ ring_k,
                                                         float *__restrict__ ring_v, int ring) {
    const int r = blockIdx.x, i = threadIdx.x;  // pair i of 256 (8 heads x 32)
    const long long pos = first + r;
    float *row = qkv + (size_t)r * 3 * kWidth;
    const float2 cs = rope[(size_t)pos * 32 + (i & 31)];
    const size_t slot = (size_t)(pos % ring) * kWidth;
#pragma unroll
    for (int part = 0; part < 2; part++) {
        float *p = row + part * kWidth + 2 * i;
        const float a = p[0], b = p[1];
        const float o0 = __fsub_rn(__fmul_rn(a, cs.x), __fmul_rn(b, cs.y));
        const float o1 = __fadd_rn(__fmul_rn(a, cs.y), __fmul_rn(b, cs.x));
        if (part == 0) {
            p[0] = o0;
            p[1] = o1;
        } else {
            ring_k[slot + 2 * i] = o0;
            ring_k[slot + 2 * i + 1] = o1;
        }
    }
    ring_v[slot + 2 * i] = row[2 * kWidth + 2 * i];
    ring_v[slot + 2 * i + 1] = row[2 * kWidth + 2 * i + 1];
}

// Windowed causal attention of one latent frame's 16 rows and one head per
// work-group: row i (position p = first + 16 f + i) attends the keys of
// positions max(0, p - context + 1) .. p. The frame's key window (at most
// context + 15 positions) goes through LDS in chunks of 64 keys: scores
// (one thread per (key, 4 rows), q . k over the 64 dimensions in order,
// times 1/8), a masked softmax per row (one wave per 4 rows), then the
// value sums (one thread per (dimension, 4 rows), keys in order), scaled
// by 1/total at the end.
constexpr int kAttnChunk = 64;
constexpr int kAttnKeys = 256 + 16;  // context <= 256, plus the frame's rows

__global__ __launch_bounds__(256) void k_mimi_attention(const float *__restrict__ qkv,
                                                        long long first,
                                                        const float *__restrict__ ring_k,
                                                        const float *__restrict__ ring_v,
                                                        int ring, int context,
                                                        float *__restrict__ out, int *status) {
    __shared__ float q[16][kHeadDim];
    __shared__ float kv[kAttnChunk][kHeadDim + 1];
    __shared__ float sc[16][kAttnKeys];
    __shared__ float totals[16];
    const int f = blockIdx.x, head = blockIdx.y, t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const long long p0 = first + 16LL * f;
    const long long kstart = p0 - (context - 1) > 0 ? p0 - (context - 1) : 0;
    const int nkeys = (int)(p0 + 16 - kstart);
    {
        const int row = t >> 4, d = (t & 15) * 4;
        const float4 v = *(const float4 *)(qkv + (size_t)(16 * f + row) * 3 * kWidth +
                                           head * kHeadDim + d);
        q[row][d] = v.x; q[row][d + 1] = v.y; q[row][d + 2] = v.z; q[row][d + 3] = v.w;
    }
    const int kk = t & 63, rg = (t >> 6) * 4;  // score / output thread roles
    for (int c0 = 0; c0 < nkeys; c0 += kAttnChunk) {
        {
            const int key = t >> 2, d = (t & 3) * 16;
            if (c0 + key < nkeys) {
                const float4 *src = (const float4 *)(ring_k + (size_t)((kstart + c0 + key) % ring) *
                                                                  kWidth + head * kHeadDim + d);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float4 v = src[u];
                    kv[key][d + 4 * u] = v.x; kv[key][d + 4 * u + 1] = v.y;
                    kv[key][d + 4 * u + 2] = v.z; kv[key][d + 4 * u + 3] = v.w;
                }
            }
        }
        __syncthreads();
        if (c0 + kk < nkeys) {
            const long long kpos = kstart + c0 + kk;
            float dot[4] = {0.f, 0.f, 0.f, 0.f};
            for (int d = 0; d < kHeadDim; d++) {
                const float kd = kv[kk][d];
#pragma unroll
                for (int i = 0; i < 4; i++) dot[i] = dot[i] + q[rg + i][d] * kd;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const long long p = p0 + rg + i;
                sc[rg + i][c0 + kk] = kpos <= p && kpos > p - context ? dot[i] * 0.125f : -INFINITY;
            }
        }
        __syncthreads();
    }
    // Masked softmax: wave w takes rows 4w .. 4w+3.
    for (int i = 0; i < 4; i++) {
        const int row = wave * 4 + i;
        float mx = -INFINITY;
        for (int j = lane; j < nkeys; j += 64) mx = fmaxf(mx, sc[row][j]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        float total = 0.0f;
        for (int j = lane; j < nkeys; j += 64) {
            const float s = sc[row][j];
            const float e = s == -INFINITY ? 0.0f : expf(s - mx);
            sc[row][j] = e;
            total += e;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) total += __shfl_xor(total, off);
        if (lane == 0) totals[row] = total;
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nkeys; c0 += kAttnChunk) {
        __syncthreads();  // scores final / previous chunk consumed
        {
            const int key = t >> 2, d = (t & 3) * 16;
            if (c0 + key < nkeys) {
                const float4 *src = (const float4 *)(ring_v + (size_t)((kstart + c0 + key) % ring) *
                                                                  kWidth + head * kHeadDim + d);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float4 v = src[u];
                    kv[key][d + 4 * u] = v.x; kv[key][d + 4 * u + 1] = v.y;
                    kv[key][d + 4 * u + 2] = v.z; kv[key][d + 4 * u + 3] = v.w;
                }
            }
        }
        __syncthreads();
        const int n = nkeys - c0 < kAttnChunk ? nkeys - c0 : kAttnChunk;
        for (int j = 0; j < n; j++) {
            const float vd = kv[j][kk];
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = acc[i] + sc[rg + i][c0 + j] * vd;
        }
    }
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float total = totals[rg + i];
        const float v = acc[i] * (1.0f / total);
        out[(size_t)(16 * f + rg + i) * kWidth + head * kHeadDim + kk] = v;
        bad |= !isfinite(v) || !(total > 0.0f);
    }
    flag_nonfinite(status, bad);
}

__device__ inline float elu1(float v) { return v <= 0.0f ? expf(v) - 1.0f : v; }

// Input row r of a convolution call: x[r] for r >= 0, else history row
// taps - 1 + r (the rows of earlier calls).
__device__ inline const float *conv_row(const float *x, const float *history, int taps, int cin,
                                        int r) {
    return r < 0 ? history + (size_t)(taps - 1 + r) * cin : x + (size_t)r * cin;
}

// The state's next history, written by the call's first work-group: the
// last `keep` rows of [history | x] (x has n rows) into `fresh`, a buffer
// that no work-group of the call reads.
__device__ inline void copy_history(const float *__restrict__ x, int n, int cin, int keep,
                                    const float *__restrict__ old, float *__restrict__ fresh) {
    if (keep <= 0 || blockIdx.x != 0 || blockIdx.y != 0 || blockIdx.z != 0) return;
    for (int i = threadIdx.x; i < keep * cin; i += blockDim.x) {
        const int row = i / cin, c = i % cin;
        const int j = n - keep + row;  // index into [history | x] relative to x
        fresh[i] = j < 0 ? old[(size_t)(keep + j) * cin + c] : x[(size_t)j * cin + c];
    }
}

// Sequential Conv1d: y[t][o] = (residual[t][o] +) (sum_{c,k} W[o][c][k]
// in(t + k - (K-1))[c] + b[o]), one thread per (t, o); w is [cin][K][cout].
__global__ __launch_bounds__(256) void k_conv_seq(const float *__restrict__ x, int positions,
                                                  int cin, int cout, int kernel,
                                                  const float *__restrict__ w,
                                                  const float *__restrict__ bias,
                                                  const float *__restrict__ history,
                                                  float *__restrict__ history_out,
                                                  const float *__restrict__ residual, int elu,
                                                  float *__restrict__ y, int *status) {
    copy_history(x, positions, cin, kernel - 1, history, history_out);
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)positions * cout) return;
    const int t = (int)(i / cout), o = (int)(i % cout);
    float dot = 0.0f;
    for (int c = 0; c < cin; c++)
        for (int k = 0; k < kernel; k++) {
            float v = conv_row(x, history, kernel, cin, t + k - (kernel - 1))[c];
            if (elu) v = elu1(v);
            dot = dot + w[((size_t)c * kernel + k) * cout + o] * v;
        }
    float out = dot + bias[o];
    if (residual) out = residual[i] + out;
    y[i] = out;
    flag_nonfinite(status, !isfinite(out));
}

// Sequential ConvTranspose1d (stride s, kernel 2s): column sums
// col(t, o, k) = sum_c W[c][o][k] in(t)[c], then y[t s + k][o] =
// (col(t, o, k) + col(t - 1, o, s + k)) + b[o]; in(-1) is the history row.
__global__ __launch_bounds__(256) void k_convtr_seq(const float *__restrict__ x, int positions,
                                                    int cin, int cout, int stride,
                                                    const float *__restrict__ w,
                                                    const float *__restrict__ bias,
                                                    const float *__restrict__ history,
                                                    float *__restrict__ history_out, int elu,
                                                    float *__restrict__ y, int *status) {
    copy_history(x, positions, cin, 1, history, history_out);
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)positions * stride * cout) return;
    const int o = (int)(i % cout), k = (int)(i / cout % stride), t = (int)(i / cout / stride);
    const int kernel = 2 * stride;
    const float *cur = x + (size_t)t * cin, *prev = conv_row(x, history, 2, cin, t - 1);
    float col = 0.0f, old = 0.0f;
    for (int c = 0; c < cin; c++) {
        const float v = elu ? elu1(cur[c]) : cur[c];
        col = col + w[((size_t)c * kernel + k) * cout + o] * v;
    }
    for (int c = 0; c < cin; c++) {
        const float v = elu ? elu1(prev[c]) : prev[c];
        old = old + w[((size_t)c * kernel + stride + k) * cout + o] * v;
    }
    const float out = (col + old) + bias[o];
    y[i] = out;
    flag_nonfinite(status, !isfinite(out));
}

// MFMA convolution (pgpu_conv_rows with fragments). A wave computes a
// 32-row x 32-column tile (columns past ncols have zero weights and are not
// stored) as 2 x 2 blocks of v_mfma_f32_16x16x32_bf16:
// A = weight fragments (16 columns x 32 reduction indices), B = 16 input
// rows x 32 channels of one tap, split into three bf16 terms (hi, mid, lo:
// exact), each term one MFMA into the same accumulator. KS = 1: the four
// waves of a work-group take four row tiles, each the whole reduction;
// KS = 4: they take quarters of the reduction of one tile and wave 0 adds
// the partial sums in wave order. Either way an output's arithmetic does
// not depend on how many rows a call has.
template <int KS>
__global__ __launch_bounds__(256) void k_conv_mfma(const float *__restrict__ x, int positions,
                                                   int cin, int cout, int taps, int ncols,
                                                   const uint16_t *__restrict__ frag,
                                                   const float *__restrict__ bias,
                                                   const float *__restrict__ history,
                                                   float *__restrict__ history_out,
                                                   const float *__restrict__ residual, int elu,
                                                   float *__restrict__ y, int *status) {
    __shared__ f32x4 part[KS > 1 ? 3 * 4 * 64 : 1];
    copy_history(x, positions, cin, taps - 1, history, history_out);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = (KS > 1 ? blockIdx.x : blockIdx.x * 4 + wave) * 32;
    const int ct0 = blockIdx.y * 2;  // first 16-column tile
    const int cbn = cin >> 5, kbn = taps * cbn;
    const int kb0 = KS > 1 ? kbn * wave / KS : 0, kb1 = KS > 1 ? kbn * (wave + 1) / KS : kbn;
    f32x4 acc[2][2];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int q = 0; q < 2; q++) acc[p][q] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool rows_live = t0 < positions;
    if (rows_live) {
        for (int kb = kb0; kb < kb1; kb++) {
            const int tap = kb / cbn, c = (kb - tap * cbn) * 32 + 8 * (lane >> 4);
            bf16x8 xs[2][3];
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const int t = t0 + p * 16 + (lane & 15);
                float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                if (t < positions) {
                    const float4 *src =
                        (const float4 *)(conv_row(x, history, taps, cin, t + tap - (taps - 1)) + c);
                    const float4 lo4 = src[0], hi4 = src[1];
                    v[0] = lo4.x; v[1] = lo4.y; v[2] = lo4.z; v[3] = lo4.w;
                    v[4] = hi4.x; v[5] = hi4.y; v[6] = hi4.z; v[7] = hi4.w;
                    if (elu) {
#pragma unroll
                        for (int e = 0; e < 8; e++) v[e] = elu1(v[e]);
                    }
                }
                uint16_t h[8], m[8], l[8];
#pragma unroll
                for (int e = 0; e < 8; e++) split3(v[e], h[e], m[e], l[e]);
                uint4 qh, qm, ql;
                qh.x = h[0] | (uint32_t)h[1] << 16; qh.y = h[2] | (uint32_t)h[3] << 16;
                qh.z = h[4] | (uint32_t)h[5] << 16; qh.w = h[6] | (uint32_t)h[7] << 16;
                qm.x = m[0] | (uint32_t)m[1] << 16; qm.y = m[2] | (uint32_t)m[3] << 16;
                qm.z = m[4] | (uint32_t)m[5] << 16; qm.w = m[6] | (uint32_t)m[7] << 16;
                ql.x = l[0] | (uint32_t)l[1] << 16; ql.y = l[2] | (uint32_t)l[3] << 16;
                ql.z = l[4] | (uint32_t)l[5] << 16; ql.w = l[6] | (uint32_t)l[7] << 16;
                xs[p][0] = __builtin_bit_cast(bf16x8, qh);
                xs[p][1] = __builtin_bit_cast(bf16x8, qm);
                xs[p][2] = __builtin_bit_cast(bf16x8, ql);
            }
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const bf16x8 wa = *(const bf16x8 *)(frag + (((size_t)(ct0 + q) * kbn + kb) * 64 +
                                                            lane) * 8);
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    acc[p][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xs[p][0], acc[p][q], 0, 0, 0);
                    acc[p][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xs[p][1], acc[p][q], 0, 0, 0);
                    acc[p][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xs[p][2], acc[p][q], 0, 0, 0);
                }
            }
        }
    }
    if constexpr (KS > 1) {
        if (wave > 0) {
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int q = 0; q < 2; q++) part[((wave - 1) * 4 + p * 2 + q) * 64 + lane] = acc[p][q];
        }
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < 3; w++)
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const f32x4 o = part[(w * 4 + p * 2 + q) * 64 + lane];
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[p][q][r] = __fadd_rn(acc[p][q][r], o[r]);
                }
    }
    if (!rows_live) return;
    bool bad = false;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int t = t0 + p * 16 + (lane & 15);
        if (t >= positions) continue;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int col = (ct0 + q) * 16 + 4 * (lane >> 4);
            if (col >= ncols) continue;
            const size_t at = (size_t)t * ncols + col;
            float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (col + r >= ncols) break;
                o[r] = __fadd_rn(acc[p][q][r], bias[(col + r) % cout]);
                if (residual) o[r] = __fadd_rn(residual[at + r], o[r]);
                bad |= !isfinite(o[r]);
            }
            if ((ncols & 3) == 0) {
                *(float4 *)(y + at) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (col + r < ncols) y[at + r] = o[r];
            }
        }
    }
    flag_nonfinite(status, bad);
}

// x <= 0 -> exp(x) - 1 (y may be x).
__global__ void k_elu(const float *__restrict__ x, float *__restrict__ y, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float v = x[i];
        y[i] = v <= 0.0f ? expf(v) - 1.0f : v;
    }
}

// One frame of the depthwise upsample (any channels <= 512, stride <= 16):
// out[o][c] = prev[c] * k[c][stride + o] + in[c] * k[c][o].
__global__ void k_upsample_frame(const float *__restrict__ kernel, const float *__restrict__ in,
                                 const float *__restrict__ prev, int channels, int stride,
                                 float *__restrict__ out, int *status) {
    const int c = threadIdx.x, o = blockIdx.x;
    if (c >= channels) return;
    const float current = in[c] * kernel[c * 2 * stride + o];
    const float old = prev[c] * kernel[c * 2 * stride + stride + o];
    const float v = old + current;
    out[o * channels + c] = v;
    flag_nonfinite(status, !isfinite(v) || !isfinite(in[c]) || !isfinite(prev[c]));
}

}  // namespace
}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_upsample_frame(void *stream, const float *kernel, const float *input,
                                   const float *previous, int channels, int stride, float *output,
                                   int *status) {
    if (!kernel || !input || !previous || !output || !status || channels <= 0 ||
        channels > 512 || stride <= 0 || stride > 16)
        return bad_arguments("pgpu_upsample_frame");
    hipLaunchKernelGGL(k_upsample_frame, dim3(stride), dim3(512), 0, (hipStream_t)stream, kernel,
                       input, previous, channels, stride, output, status);
    return launch_ok("pgpu_upsample_frame");
}

extern "C" int pgpu_mimi_input(void *stream, const float *latents, int frames,
                               const float *projection, const float *upsample, float *previous,
                               float *hidden, int *status) {
    if (!latents || frames <= 0 || frames > 65535 || !projection || !upsample || !previous ||
        !hidden || !status)
        return bad_arguments("pgpu_mimi_input");
    hipLaunchKernelGGL(k_mimi_input, dim3(frames, kWidth / 256), dim3(256), 0,
                       (hipStream_t)stream, latents, frames, projection, upsample, previous,
                       hidden, status);
    hipLaunchKernelGGL(k_mimi_keep_previous, dim3(kWidth / 256), dim3(256), 0,
                       (hipStream_t)stream, latents, frames - 1, projection, previous);
    return launch_ok("pgpu_mimi_input");
}

extern "C" int pgpu_mimi_rope_store(void *stream, float *qkv, int rows, long long first,
                                    const float *rope, long long rope_positions, float *ring_k,
                                    float *ring_v, int ring) {
    if (!qkv || rows <= 0 || rows > 65535 || first < 0 || !rope ||
        first + rows > rope_positions || !ring_k || !ring_v || ring < rows)
        return bad_arguments("pgpu_mimi_rope_store");
    hipLaunchKernelGGL(k_mimi_rope_store, dim3(rows), dim3(256), 0, (hipStream_t)stream, qkv,
                       rows, first, (const float2 *)rope, ring_k, ring_v, ring);
    return launch_ok("pgpu_mimi_rope_store");
}

extern "C" int pgpu_mimi_attention(void *stream, const float *qkv, int rows, long long first,
                                   const float *ring_k, const float *ring_v, int ring,
                                   int context, float *out, int *status) {
    if (!qkv || rows <= 0 || rows % 16 || rows > 65535 || first < 0 || !ring_k || !ring_v ||
        context <= 0 || context > 256 || ring < rows + context - 1 || !out || !status)
        return bad_arguments("pgpu_mimi_attention");
    hipLaunchKernelGGL(k_mimi_attention, dim3(rows / 16, kHeads), dim3(256), 0,
                       (hipStream_t)stream, qkv, first, ring_k, ring_v, ring, context, out, status);
    return launch_ok("pgpu_mimi_attention");
}

extern "C" int pgpu_conv_rows(void *stream, const pgpu_conv_layer *L, const float *x,
                              int positions, const float *history, float *history_out,
                              const float *residual, int elu, float *y, int *status) {
    if (!L || !x || positions <= 0 || !y || !status || L->cin <= 0 || L->cin > 512 ||
        L->cout <= 0 || L->cout > 512 || !L->bias)
        return bad_arguments("pgpu_conv_rows");
    const bool tr = L->transpose != 0;
    const bool shape_ok = tr ? (L->stride >= 4 && L->stride <= 6 && L->kernel == 2 * L->stride &&
                                L->taps == 2 && L->ncols == L->stride * L->cout)
                             : (L->stride == 1 && (L->kernel == 1 || L->kernel == 3 ||
                                                   L->kernel == 7) &&
                                L->taps == L->kernel && L->ncols == L->cout);
    const size_t outs = (size_t)positions * L->ncols;
    if (!shape_ok || (L->taps > 1 && (!history || !history_out)) ||
        (tr && residual) || (L->fragments && L->cin % 32) ||
        (!L->fragments && !L->weight) || outs > (size_t)0x7fffffff)
        return bad_arguments("pgpu_conv_rows");
    hipStream_t st = (hipStream_t)stream;
    if (L->fragments) {
        const int kbn = L->taps * L->cin / 32, tiles = (positions + 31) / 32;
        const int col_tiles = (L->ncols + 31) / 32;
        if (kbn >= 16)
            hipLaunchKernelGGL(k_conv_mfma<4>, dim3(tiles, col_tiles), dim3(256), 0, st, x,
                               positions, L->cin, L->cout, L->taps, L->ncols, L->fragments,
                               L->bias, history, history_out, residual, elu, y, status);
        else
            hipLaunchKernelGGL(k_conv_mfma<1>, dim3((tiles + 3) / 4, col_tiles), dim3(256), 0,
                               st, x, positions, L->cin, L->cout, L->taps, L->ncols, L->fragments,
                               L->bias, history, history_out, residual, elu, y, status);
    } else if (tr) {
        hipLaunchKernelGGL(k_convtr_seq, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st,
                           x, positions, L->cin, L->cout, L->stride, L->weight, L->bias, history,
                           history_out, elu, y, status);
    } else {
        hipLaunchKernelGGL(k_conv_seq, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st, x,
                           positions, L->cin, L->cout, L->kernel, L->weight, L->bias, history,
                           history_out, residual, elu, y, status);
    }
    return launch_ok("pgpu_conv_rows");
}

extern "C" int pgpu_elu(void *stream, const float *x, float *y, size_t count) {
    if (!x || !y || !count) return bad_arguments("pgpu_elu");
    const unsigned blocks = (unsigned)((count + 255) / 256 < 4096 ? (count + 255) / 256 : 4096);
    hipLaunchKernelGGL(k_elu, dim3(blocks), dim3(256), 0, (hipStream_t)stream, x, y, count);
    return launch_ok("pgpu_elu");
}
