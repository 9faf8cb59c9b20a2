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

// Windowed causal attention: one wave per (row, head). Row r (position
// p = first + r) attends the keys of positions max(0, p - context + 1) .. p.
// Lane j scores keys j, j + 64, ...; the exponentials go through LDS and
// lane d accumulates output dimension d.
__global__ __launch_bounds__(64) void k_mimi_attention(const float *__restrict__ qkv,
                                                       long long first,
                                                       const float *__restrict__ ring_k,
                                                       const float *__restrict__ ring_v, int ring,
                                                       int context, float *__restrict__ out,
                                                       int *status) {
    __shared__ float weights[256];
    __shared__ float q[kHeadDim];
    const int r = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    const long long pos = first + r;
    const int count = (int)(pos + 1 < context ? pos + 1 : context);
    const long long start = pos + 1 - count;
    q[lane] = qkv[(size_t)r * 3 * kWidth + head * kHeadDim + lane];
    __syncthreads();
    float mx = -INFINITY;
    float s[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int key = lane + 64 * u;
        s[u] = -INFINITY;
        if (key < count) {
            const float *k = ring_k + (size_t)((start + key) % ring) * kWidth + head * kHeadDim;
            float dot = 0.0f;
#pragma unroll 8
            for (int d = 0; d < kHeadDim; d++) dot = dot + q[d] * k[d];
            s[u] = dot * 0.125f;
            mx = fmaxf(mx, s[u]);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float total = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int key = lane + 64 * u;
        if (key < count) {
            const float e = expf(s[u] - mx);
            weights[key] = e;
            total += e;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) total += __shfl_xor(total, off);
    __syncthreads();
    float acc = 0.0f;
    for (int key = 0; key < count; key++)
        acc = acc + weights[key] * ring_v[(size_t)((start + key) % ring) * kWidth + head * kHeadDim + lane];
    const float v = acc * (1.0f / total);
    out[(size_t)r * kWidth + head * kHeadDim + lane] = v;
    flag_nonfinite(status, !isfinite(v) || !(total > 0.0f) || !isfinite(mx));
}

// Causal Conv1d: y[t][o] = (sum_{c,k} W[o][c][k] in[t + k - (K-1)][c]) + b[o]
// (+ residual[t][o] first when given: y = residual + (dot + b)). w is
// [cin][K][cout]; in[j] for j < 0 is history row K - 1 + j ([K-1][cin]).
__global__ __launch_bounds__(256) void k_conv1d(const float *__restrict__ x, int cin, int cout,
                                                int kernel, const float *__restrict__ w,
                                                const float *__restrict__ bias,
                                                const float *__restrict__ history,
                                                const float *__restrict__ residual,
                                                float *__restrict__ y, int *status) {
    const int t = blockIdx.x, o = blockIdx.y * 256 + threadIdx.x;
    if (o >= cout) return;
    float dot = 0.0f;
    for (int c = 0; c < cin; c++)
        for (int k = 0; k < kernel; k++) {
            const int j = t + k - (kernel - 1);
            const float v = j < 0 ? history[(size_t)(kernel - 1 + j) * cin + c] : x[(size_t)j * cin + c];
            dot = dot + w[((size_t)c * kernel + k) * cout + o] * v;
        }
    float out = dot + bias[o];
    if (residual) out = residual[(size_t)t * cout + o] + out;
    y[(size_t)t * cout + o] = out;
    flag_nonfinite(status, !isfinite(out));
}

// New history: the last K-1 rows of [history | x] (positions n).
__global__ void k_conv_history(const float *__restrict__ x, int n, int cin, int keep,
                               const float *__restrict__ old, float *__restrict__ fresh) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)keep * cin) return;
    const int row = (int)(i / cin), c = (int)(i % cin);
    const int j = n - keep + row;  // index into [history | x] relative to x
    fresh[i] = j < 0 ? old[(size_t)(keep + j) * cin + c] : x[(size_t)j * cin + c];
}

// Causal ConvTranspose1d (stride s, kernel 2s): column (t, o, k) =
// sum_c W[c][o][k] x[t][c]; y[t s + k][o] = (col(t, o, k) + col(t-1, o, s+k))
// + b[o], col(-1, .) being the state's overlap. w is [cin][2s][cout].
__global__ __launch_bounds__(256) void k_convtr1d(const float *__restrict__ x, int cin, int cout,
                                                  int stride, const float *__restrict__ w,
                                                  const float *__restrict__ bias,
                                                  const float *__restrict__ overlap,
                                                  float *__restrict__ y, int *status) {
    const int t = blockIdx.x, k = blockIdx.z, o = blockIdx.y * 256 + threadIdx.x;
    if (o >= cout) return;
    const int kernel = 2 * stride;
    float col = 0.0f;
    for (int c = 0; c < cin; c++)
        col = col + w[((size_t)c * kernel + k) * cout + o] * x[(size_t)t * cin + c];
    float prev;
    if (t == 0) {
        prev = overlap[(size_t)k * cout + o];
    } else {
        prev = 0.0f;
        for (int c = 0; c < cin; c++)
            prev = prev + w[((size_t)c * kernel + stride + k) * cout + o] * x[(size_t)(t - 1) * cin + c];
    }
    const float out = (col + prev) + bias[o];
    y[((size_t)t * stride + k) * cout + o] = out;
    flag_nonfinite(status, !isfinite(out));
}

// The overlap the next call starts from: col(n - 1, o, s + k).
__global__ __launch_bounds__(256) void k_convtr_tail(const float *__restrict__ x, int n, int cin,
                                                     int cout, int stride,
                                                     const float *__restrict__ w,
                                                     float *__restrict__ overlap) {
    const int k = blockIdx.x, o = blockIdx.y * 256 + threadIdx.x;
    if (o >= cout) return;
    const int kernel = 2 * stride;
    float col = 0.0f;
    for (int c = 0; c < cin; c++)
        col = col + w[((size_t)c * kernel + stride + k) * cout + o] * x[(size_t)(n - 1) * cin + c];
    overlap[(size_t)k * cout + o] = col;
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
    if (!qkv || rows <= 0 || rows > 65535 || first < 0 || !ring_k || !ring_v || context <= 0 ||
        context > 256 || ring < rows + context - 1 || !out || !status)
        return bad_arguments("pgpu_mimi_attention");
    hipLaunchKernelGGL(k_mimi_attention, dim3(rows, kHeads), dim3(64), 0, (hipStream_t)stream,
                       qkv, first, ring_k, ring_v, ring, context, out, status);
    return launch_ok("pgpu_mimi_attention");
}

extern "C" int pgpu_conv1d(void *stream, const float *x, int positions, int cin, int cout,
                           int kernel, const float *weight, const float *bias,
                           const float *history, float *history_out, const float *residual,
                           float *y, int *status) {
    if (!x || positions <= 0 || positions > 65535 || cin <= 0 || cin > 512 || cout <= 0 ||
        cout > 512 || (kernel != 1 && kernel != 3 && kernel != 7) || !weight || !bias ||
        (kernel > 1 && (!history || !history_out)) || !y || !status)
        return bad_arguments("pgpu_conv1d");
    hipLaunchKernelGGL(k_conv1d, dim3(positions, (cout + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, x, cin, cout, kernel, weight, bias, history, residual,
                       y, status);
    if (kernel > 1) {
        const size_t n = (size_t)(kernel - 1) * cin;
        hipLaunchKernelGGL(k_conv_history, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           (hipStream_t)stream, x, positions, cin, kernel - 1, history,
                           history_out);
    }
    return launch_ok("pgpu_conv1d");
}

extern "C" int pgpu_convtr1d(void *stream, const float *x, int positions, int cin, int cout,
                             int stride, const float *weight, const float *bias, float *overlap,
                             float *y, int *status) {
    if (!x || positions <= 0 || positions > 65535 || cin <= 0 || cin > 512 || cout <= 0 ||
        cout > 512 || stride < 4 || stride > 6 || !weight || !bias || !overlap || !y || !status)
        return bad_arguments("pgpu_convtr1d");
    hipLaunchKernelGGL(k_convtr1d, dim3(positions, (cout + 255) / 256, stride), dim3(256), 0,
                       (hipStream_t)stream, x, cin, cout, stride, weight, bias, overlap, y,
                       status);
    hipLaunchKernelGGL(k_convtr_tail, dim3(stride, (cout + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, x, positions, cin, cout, stride, weight, overlap);
    return launch_ok("pgpu_convtr1d");
}

extern "C" int pgpu_elu(void *stream, const float *x, float *y, size_t count) {
    if (!x || !y || !count) return bad_arguments("pgpu_elu");
    const unsigned blocks = (unsigned)((count + 255) / 256 < 4096 ? (count + 255) / 256 : 4096);
    hipLaunchKernelGGL(k_elu, dim3(blocks), dim3(256), 0, (hipStream_t)stream, x, y, count);
    return launch_ok("pgpu_elu");
}
