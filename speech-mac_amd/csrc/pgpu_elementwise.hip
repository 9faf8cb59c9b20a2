// Row and element kernels of the decode step: LayerNorm into split
// fragments, the standalone norm/GELU/RoPE primitives of the C API, and KV
// pool data movement (row append, paged <-> contiguous copies, synthetic fill).
#include "pgpu_common.hpp"
#include "phonon_gpu.h"

namespace pgpu {

// LayerNorm of 512-wide rows, one wave per stream, written as split
// fragments for the next projection (and optionally as fp32).
// Replaces phonon_layer_norm at width 512 (src/phonon_transformer.c:153-185):
// two-pass fp32 moments instead of the reference's Welford cascade; output
// y = ((x - mean) * rstd) * w + b, unfused like the reference.
__global__ __launch_bounds__(256) void k_ln_split(const float *__restrict__ x, int streams,
                                                  const float *__restrict__ w,
                                                  const float *__restrict__ b, float eps,
                                                  uint16_t *__restrict__ xs,
                                                  float *__restrict__ y, int *status) {
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
        const float c = v[i] - mean;
        sq = fmaf(c, c, sq);
    }
    const float var = wave_sum(sq) * (1.0f / kWidth);
    const float rstd = 1.0f / sqrtf(var + eps);
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int k = lane * 8 + i;
        v[i] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i], mean), rstd), w[k]), b[k]);
        bad |= !isfinite(v[i]);
    }
    if (xs) store_split<8>(xs, s, lane * 8, kWidth / 32, v);
    if (y) {
        float *o = y + (size_t)s * kWidth + lane * 8;
        *(float4 *)o = make_float4(v[0], v[1], v[2], v[3]);
        *(float4 *)(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    flag_nonfinite(status, bad);
}

// fp32 rows [streams][k_cols] -> split fragments (k_cols % 256 == 0).
__global__ __launch_bounds__(256) void k_split_rows(const float *__restrict__ x, int streams,
                                                   int k_cols, uint16_t *__restrict__ xs,
                                                   int *status) {
    const int groups = k_cols / 8;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int s = (int)(i / groups), g = (int)(i % groups);
    bool bad = false;
    if (s < streams) {
        const float *row = x + (size_t)s * k_cols + g * 8;
        const float4 a0 = *(const float4 *)row, a1 = *(const float4 *)(row + 4);
        float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) bad |= !isfinite(v[j]);
        store_split<8>(xs, s, g * 8, k_cols / 32, v);
    }
    flag_nonfinite(status, bad);
}

// Block-wide double sum over 256 threads.
__device__ inline double block_sum_f64(double v, double *shared) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) shared[wave] = v;
    __syncthreads();
    return shared[0] + shared[1] + shared[2] + shared[3];
}

// One row of any width: LayerNorm (mode 0) or RMSNorm (mode 1) with double
// moments, as the reference computes them for widths other than 512
// (src/phonon_transformer.c:66-85, 168-178).
__global__ __launch_bounds__(256) void k_norm_row(const float *__restrict__ x, int width,
                                                  const float *__restrict__ w,
                                                  const float *__restrict__ b, float eps,
                                                  int mode, float *__restrict__ y,
                                                  int *status) {
    __shared__ double shared[4];
    double sum = 0.0, sq = 0.0;
    for (int i = threadIdx.x; i < width; i += 256) {
        sum += x[i];
        sq += (double)x[i] * x[i];
    }
    sum = block_sum_f64(sum, shared);
    sq = block_sum_f64(sq, shared);
    bool bad = false;
    if (mode == 1) {
        const float scale = 1.0f / sqrtf(__fadd_rn((float)(sq / width), eps));
        for (int i = threadIdx.x; i < width; i += 256) {
            y[i] = __fmul_rn(__fmul_rn(x[i], scale), w[i]);
            bad |= !isfinite(y[i]);
        }
    } else {
        const double mean = sum / width;
        double cs = 0.0;
        for (int i = threadIdx.x; i < width; i += 256) {
            const double c = (double)x[i] - mean;
            cs += c * c;
        }
        cs = block_sum_f64(cs, shared);
        const float scale = 1.0f / sqrtf(__fadd_rn((float)(cs / width), eps));
        for (int i = threadIdx.x; i < width; i += 256) {
            const float c = (float)((double)x[i] - mean);
            y[i] = __fadd_rn(__fmul_rn(__fmul_rn(c, scale), w[i]), b[i]);
            bad |= !isfinite(y[i]);
        }
    }
    flag_nonfinite(status, bad);
}

// Exact GELU of src/phonon_transformer.c:202-216: polynomial erf on full
// groups of four, device erff on the count%4 tail.
__global__ __launch_bounds__(256) void k_gelu(float *__restrict__ v, size_t count,
                                              int *status) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    bool bad = false;
    if (i < count) {
        const float x = v[i];
        float g;
        if (i < count - count % 4) {
            g = gelu_erf(x);
        } else {
            const float e = erff(__fmul_rn(x, 0.7071067811865475244f));
            g = __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, e));
        }
        bad = !isfinite(x) || !isfinite(g);
        v[i] = g;
    }
    flag_nonfinite(status, bad);
}

// Interleaved RoPE of one vector of `heads` heads of `head_width`, with
// (cos, sin) per pair precomputed by the host (src/phonon_transformer.c:218-251).
__global__ __launch_bounds__(256) void k_rope(float *__restrict__ v, int heads, int head_width,
                                              const float2 *__restrict__ cs, int *status) {
    const int half = head_width / 2;
    const int i = blockIdx.x * 256 + threadIdx.x;
    bool bad = false;
    if (i < heads * half) {
        const int h = i / half, p = i % half;
        float *pair = v + h * head_width + 2 * p;
        const float a = pair[0], b = pair[1];
        const float2 c = cs[p];
        pair[0] = __fsub_rn(__fmul_rn(a, c.x), __fmul_rn(b, c.y));
        pair[1] = __fadd_rn(__fmul_rn(a, c.y), __fmul_rn(b, c.x));
        bad = !isfinite(a) || !isfinite(b) || !isfinite(pair[0]) || !isfinite(pair[1]);
    }
    flag_nonfinite(status, bad);
}

// Paged <-> contiguous copies for one stream. Contiguous rows follow the
// reference cache layout [layer][capacity][512] (src/phonon_transformer.c:53):
// `keys`/`values` point at the row of (first_layer, first_position) and the
// row of (first_layer + y, first_position + x) is `capacity*y + x` rows
// further. direction 0: contiguous -> pool, 1: pool -> contiguous.
// Grid (count, layers).
__global__ __launch_bounds__(128) void k_kv_copy(float *__restrict__ pool, size_t layer_stride,
                                                 unsigned blocks, const int32_t *__restrict__ table,
                                                 int first_position, int first_layer,
                                                 float *__restrict__ keys,
                                                 float *__restrict__ values, size_t capacity,
                                                 int direction, int *status) {
    const int pos = first_position + blockIdx.x, layer = first_layer + blockIdx.y;
    const int block = table[pos >> 4];
    if ((unsigned)block >= blocks) {
        if (threadIdx.x == 0) atomicOr(status, 2);
        return;
    }
    const int c = threadIdx.x * 4, head = c >> 6, d = c & 63;
    float *tile = pool + (size_t)layer * layer_stride + ((size_t)block * kHeads + head) * 2048 +
                  (pos & 15) * 64 + d;
    const size_t row = ((size_t)blockIdx.y * capacity + blockIdx.x) * kWidth + c;
    if (direction == 0) {
        *(float4 *)tile = *(const float4 *)(keys + row);
        *(float4 *)(tile + 1024) = *(const float4 *)(values + row);
    } else {
        *(float4 *)(keys + row) = *(const float4 *)tile;
        *(float4 *)(values + row) = *(const float4 *)(tile + 1024);
    }
}

__device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Deterministic N(0,1) fill (counter-hash uniform pairs + Box-Muller).
__global__ __launch_bounds__(256) void k_fill_normal(float *__restrict__ dst, size_t pairs,
                                                     size_t first_pair, uint64_t seed) {
    const size_t i = first_pair + (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pairs) return;
    const uint64_t r = mix64(seed ^ mix64(i));
    const float u1 = ((uint32_t)(r >> 40) + 1) * (1.0f / 16777217.0f);
    const float u2 = (uint32_t)(r & 0xffffff) * (1.0f / 16777216.0f);
    const float rad = sqrtf(-2.0f * logf(u1));
    float sn, cn;
    sincosf(6.283185307179586f * u2, &sn, &cn);
    *(float2 *)(dst + 2 * i) = make_float2(rad * cn, rad * sn);
}

__global__ void k_advance(int32_t *positions, int streams, int delta) {
    const int s = blockIdx.x * 256 + threadIdx.x;
    if (s < streams) positions[s] += delta;
}

__global__ void k_fill_u32(uint32_t *dst, size_t n, uint32_t value) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = value;
}

// dst row r = src row map[r] (int32 rows of `width`): per-token copies of a
// stream's block table for a batched prefill. Grid (ceil(width/256), rows).
// Row r of dst = row map[r] of src; with copy_dst, also copy_dst[r] =
// copy_src[r] (one value per row, by the row's first work-group).
__global__ void k_gather_rows(int32_t *__restrict__ dst, const int32_t *__restrict__ src,
                              const int32_t *__restrict__ map, int width,
                              int32_t *__restrict__ copy_dst,
                              const int32_t *__restrict__ copy_src) {
    const int i = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (i < width) dst[(size_t)r * width + i] = src[(size_t)map[r] * width + i];
    if (copy_dst && i == 0) copy_dst[r] = copy_src[r];
}

}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_ln_split(void *stream, const float *x, int streams, const float *w,
                             const float *b, float eps, uint16_t *xs, float *y, int *status) {
    if (streams <= 0 || (!xs && !y)) return bad_arguments(__func__);
    hipLaunchKernelGGL(k_ln_split, dim3((streams + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       x, streams, w, b, eps, xs, y, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_split_rows(void *stream, const float *x, int streams, int k_cols,
                               uint16_t *xs, int *status) {
    if (streams <= 0 || k_cols <= 0 || k_cols % 32) return bad_arguments(__func__);
    const size_t threads = (size_t)streams * (k_cols / 8);
    hipLaunchKernelGGL(k_split_rows, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, x, streams, k_cols, xs, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_norm_row(void *stream, const float *x, int width, const float *w,
                             const float *b, float eps, int rms, float *y, int *status) {
    if (width <= 0) return bad_arguments(__func__);
    hipLaunchKernelGGL(k_norm_row, dim3(1), dim3(256), 0, (hipStream_t)stream, x, width, w, b,
                       eps, rms, y, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_gelu(void *stream, float *values, size_t count, int *status) {
    if (!count) return 1;
    hipLaunchKernelGGL(k_gelu, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, values, count, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_rope(void *stream, float *values, int heads, int head_width,
                         const float *cos_sin, int *status) {
    if (heads <= 0 || head_width <= 0 || head_width % 2) return bad_arguments(__func__);
    const int pairs = heads * head_width / 2;
    hipLaunchKernelGGL(k_rope, dim3((pairs + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       values, heads, head_width, (const float2 *)cos_sin, status);
    return launch_ok(__func__);
}

extern "C" int pgpu_kv_copy(void *stream, const pgpu_paged_kv *kv, const int32_t *table,
                            int first_position, int count, int first_layer, int layers,
                            float *keys, float *values, size_t capacity, int to_contiguous,
                            int *status) {
    if (count <= 0 || layers <= 0 || first_layer < 0 || first_layer + layers > kv->layers ||
        first_position < 0 || (layers > 1 && (size_t)count > capacity))
        return bad_arguments(__func__);
    hipLaunchKernelGGL(k_kv_copy, dim3(count, layers), dim3(128), 0, (hipStream_t)stream,
                       kv->base, kv->layer_stride, (unsigned)kv->blocks, table, first_position,
                       first_layer, keys, values, capacity, to_contiguous ? 1 : 0, status);
    return launch_ok(__func__);
}

// A dispatch packet counts work-items in 32 bits (grid_size_x), so one
// dispatch of this kernel covers at most PGPU_FILL_MAX_GROUPS work-groups of
// 256 work-items (2^31 pairs): a 103 GB pool is 12.9 G pairs, i.e. 6
// dispatches. Dispatch i fills pairs [first, first + pairs).
extern "C" size_t pgpu_fill_normal_plan(size_t count, size_t i, size_t *first, size_t *pairs) {
    const size_t total = count / 2, per = (size_t)PGPU_FILL_MAX_GROUPS * 256;
    const size_t n = (total + per - 1) / per;
    if (i < n && first && pairs) {
        *first = i * per;
        *pairs = total - i * per < per ? total - i * per : per;
    }
    return n;
}

extern "C" int pgpu_fill_normal(void *stream, float *dst, size_t count, uint64_t seed) {
    if (!dst || count % 2) return bad_arguments(__func__);
    const size_t n = pgpu_fill_normal_plan(count, 0, nullptr, nullptr);
    for (size_t i = 0; i < n; i++) {
        size_t first = 0, pairs = 0;
        pgpu_fill_normal_plan(count, i, &first, &pairs);
        const unsigned groups = (unsigned)((pairs + 255) / 256);
        hipLaunchKernelGGL(k_fill_normal, dim3(groups), dim3(256), 0, (hipStream_t)stream, dst,
                           first + pairs, first, seed);
        if (!launch_ok(__func__)) return 0;
    }
    return 1;
}

extern "C" int pgpu_advance_positions(void *stream, int32_t *positions, int streams, int delta) {
    if (!positions || streams <= 0) return bad_arguments(__func__);
    hipLaunchKernelGGL(k_advance, dim3((streams + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, positions, streams, delta);
    return launch_ok(__func__);
}

extern "C" int pgpu_gather_rows_copy(void *stream, int32_t *dst, const int32_t *src,
                                     const int32_t *map, int rows, int width, int32_t *copy_dst,
                                     const int32_t *copy_src) {
    if (!dst || !src || !map || rows <= 0 || width <= 0 || !copy_dst != !copy_src)
        return bad_arguments(__func__);
    hipLaunchKernelGGL(k_gather_rows, dim3((width + 255) / 256, rows), dim3(256), 0,
                       (hipStream_t)stream, dst, src, map, width, copy_dst, copy_src);
    return launch_ok(__func__);
}

extern "C" int pgpu_gather_rows(void *stream, int32_t *dst, const int32_t *src,
                                const int32_t *map, int rows, int width) {
    return pgpu_gather_rows_copy(stream, dst, src, map, rows, width, nullptr, nullptr);
}

extern "C" int pgpu_fill_u32(void *stream, uint32_t *dst, size_t n, uint32_t value) {
    if (!dst || !n) return bad_arguments(__func__);
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, dst, n, value);
    return launch_ok(__func__);
}
