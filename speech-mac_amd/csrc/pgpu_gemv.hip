// Small-batch Q8_0 matrix-vector products on the vector units: y[s][r] =
// sum over 32-column blocks b of scale[r][b] * partial(r, b, s), with
// partial = sum_i (float)q[r][32b + i] * x[s][32b + i] (src/phonon_q8.c:36-62).
//
// One lane per (row, block): its 32 int8 weights arrive in two 16-byte
// loads from a row-major copy of the matrix, its scale from a separate
// fp16 plane. The lane forms the block's partial with the reference's
// arithmetic (each product rounded to fp32, then added, in column order)
// and scales it; the row's first lane then adds the rows' scaled partials
// in block order. The result therefore has the bits of the reference's
// phonon_q8_matvec compiled without multiply-add contraction
// (-ffp-contract=off, as its golden vectors here are built). The
// reference's own build (clang, no contraction flag) may contract
// `partial += (float)q * x` and `sum += scale * partial` into fused
// multiply-adds, whose results can differ in the last bits: against such a
// build the outputs agree within the fp32 tolerance, not bit for bit. A wave
// holds 64 / (columns / 32) whole rows, so the columns must be 32 times a
// divisor of 64 (32 .. 2048).
#include "pgpu_gemm.hpp"
#include "phonon_gpu.h"

namespace pgpu {
namespace {

template <int B>
__global__ __launch_bounds__(64) void k_q8_gemv(const int8_t *__restrict__ values,
                                                const uint16_t *__restrict__ scales, int rows,
                                                int columns, const float *__restrict__ x,
                                                float *__restrict__ y, int *status) {
    const int nb = columns >> 5, per_wave = 64 / nb;
    const int lane = threadIdx.x;
    const int r_in = lane / nb, b = lane - r_in * nb;
    const int row = blockIdx.x * per_wave + r_in;
    const bool live = row < rows;
    float scaled[B];
    bool bad = false;
#pragma unroll
    for (int s = 0; s < B; s++) scaled[s] = 0.0f;
    if (live) {
        const int4 *w = (const int4 *)(values + (size_t)row * columns + b * 32);
        const int4 w0 = w[0], w1 = w[1];
        const int words[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float q[32];
#pragma unroll
        for (int i = 0; i < 32; i++) q[i] = (float)(int8_t)(words[i >> 2] >> (8 * (i & 3)));
        const float scale = half_to_float(scales[(size_t)row * nb + b]);
        bad |= !isfinite(scale);
#pragma unroll
        for (int s = 0; s < B; s++) {
            const float4 *xv = (const float4 *)(x + (size_t)s * columns + b * 32);
            float partial = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 v = xv[i];
                bad |= !isfinite(v.x) || !isfinite(v.y) || !isfinite(v.z) || !isfinite(v.w);
                partial = __fadd_rn(partial, __fmul_rn(q[4 * i], v.x));
                partial = __fadd_rn(partial, __fmul_rn(q[4 * i + 1], v.y));
                partial = __fadd_rn(partial, __fmul_rn(q[4 * i + 2], v.z));
                partial = __fadd_rn(partial, __fmul_rn(q[4 * i + 3], v.w));
            }
            scaled[s] = __fmul_rn(scale, partial);
        }
    }
    // The row's scaled partials added in block order (every lane of the row
    // forms the same sum; the first one stores it).
#pragma unroll
    for (int s = 0; s < B; s++) {
        float sum = 0.0f;
        for (int j = 0; j < nb; j++) sum = __fadd_rn(sum, __shfl(scaled[s], r_in * nb + j));
        if (live && b == 0) {
            y[(size_t)s * rows + row] = sum;
            bad |= !isfinite(sum);
        }
    }
    flag_nonfinite(status, bad && live);
}

}  // namespace
}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_q8_gemv(void *stream, const int8_t *values, const uint16_t *scales, int rows,
                            int columns, const float *x, int batch, float *y, int *status) {
    const int nb = columns / 32;
    if (!values || !scales || !x || !y || !status || rows <= 0 || columns < 32 ||
        columns % 32 || nb > 64 || 64 % nb || batch < 1 || batch > PGPU_GEMV_MAX_BATCH ||
        (uintptr_t)values % 16 || (uintptr_t)x % 16)
        return bad_arguments("pgpu_q8_gemv");
    const int per_wave = 64 / nb;
    const dim3 grid((unsigned)((rows + per_wave - 1) / per_wave));
    hipStream_t st = (hipStream_t)stream;
    switch (batch) {
    case 1: hipLaunchKernelGGL(k_q8_gemv<1>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    case 2: hipLaunchKernelGGL(k_q8_gemv<2>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    case 3: hipLaunchKernelGGL(k_q8_gemv<3>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    case 4: hipLaunchKernelGGL(k_q8_gemv<4>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    case 5: hipLaunchKernelGGL(k_q8_gemv<5>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    case 6: hipLaunchKernelGGL(k_q8_gemv<6>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    case 7: hipLaunchKernelGGL(k_q8_gemv<7>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    default: hipLaunchKernelGGL(k_q8_gemv<8>, grid, dim3(64), 0, st, values, scales, rows, columns, x, y, status); break;
    }
    return launch_ok("pgpu_q8_gemv");
}
