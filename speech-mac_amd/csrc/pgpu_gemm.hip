// Projection kernel of the decode step: Y[s][n] = sum_k X[s][k] * W[n][k]
// for B streams, on v_mfma_f32_16x16x32_bf16.
//
// Replaces the fp32 SGEMM of phonon_linear (src/phonon_transformer.c:253-313)
// and the row dot of phonon_q8_matvec (src/phonon_q8.c:36-92).
//
// Operands
//   W  Q8_0: int8 values in MFMA A-fragment order, one 512-byte record per
//      (16-row tile, 32-column block); lane l holds row l%16, columns
//      8*(l/16) .. +7. The per-(row, block) fp16 scales sit in a separate
//      plane [tile][block][16]. Bytes per weight: 1 + 2/32 (same as Q8_0).
//   W  BF16: the same fragment order with bf16 values (1024-byte records).
//   X  split fragments (pgpu_common.hpp): three bf16 terms per activation.
// Arithmetic
//   Q8: per 32-column block, c = W_q8 . (X_hi + X_mid + X_lo) by three MFMAs
//   from zero (int8 and bf16 terms multiply exactly), then acc += scale*c,
//   i.e. the reference phonon_q8_dot order "sum += scale * partial".
//   BF16: the three MFMAs chain straight into the accumulator.
// Work decomposition
//   One work-group = 16 output rows x 16 streams; its 4 waves split the
//   column blocks into 4 contiguous ranges and are summed in LDS in wave
//   order, so results do not depend on scheduling.
#include <hip/hip_fp16.h>

#include "pgpu_common.hpp"
#include "phonon_gpu.h"

namespace pgpu {

enum Epilogue { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_GELU_SPLIT = 2, EPI_QKV = 3 };

struct GemmArgs {
    const uint16_t *xs;       // split-fragment input, k_cols/32 blocks per row
    const void *w;            // weight fragments
    const uint16_t *wscale;   // Q8 only
    int n_rows, k_cols, streams;
    float *out;               // STORE / RESIDUAL: [streams][ld_out]
    int ld_out;
    const float *bias;        // STORE: optional [n_rows]
    const float *residual;    // RESIDUAL: [streams][ld_out]
    uint16_t *out_split;      // GELU_SPLIT: split fragments with out_kb blocks per row
    int out_kb;
    float *q_out;             // QKV: [streams][512]
    float *kv;                // QKV: paged pool base
    size_t layer_stride;      // floats per layer of the pool
    unsigned blocks;          // QKV: blocks per layer of the pool
    int layer;
    const int32_t *tables;
    int table_stride;
    const int32_t *positions;
    const float2 *rope;       // [8192][32] (cos, sin)
    int *status;
};

__device__ inline bf16x8 q8_to_bf16(uint2 raw) {
    typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
    u32x4 packed;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t word = i < 2 ? raw.x : raw.y;
        const int shift = (i & 1) * 16;
        const float f0 = (float)(int8_t)(word >> shift);
        const float f1 = (float)(int8_t)(word >> (shift + 8));
        packed[i] = (fbits(f0) >> 16) | (fbits(f1) & 0xffff0000u);
    }
    return __builtin_bit_cast(bf16x8, packed);
}

__device__ inline float half_to_float(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)bits16));
}

template <int EPI, bool Q8>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
    const int tile = blockIdx.x, st = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kbn = a.k_cols >> 5;
    const int per_wave = (kbn + 3) >> 2;
    const int kb_begin = wave * per_wave;
    const int kb_end = min(kbn, kb_begin + per_wave);

    const uint16_t *xs = a.xs + (size_t)st * kbn * 1536 + lane * 8;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (Q8) {
        const int8_t *wq = (const int8_t *)a.w + (size_t)tile * kbn * 512 + lane * 8;
        const uint16_t *ws = a.wscale + (size_t)tile * kbn * 16 + (lane >> 4) * 4;
        for (int kb = kb_begin; kb < kb_end; kb++) {
            const bf16x8 wa = q8_to_bf16(*(const uint2 *)(wq + (size_t)kb * 512));
            const uint2 sc = *(const uint2 *)(ws + (size_t)kb * 16);
            const bf16x8 xh = *(const bf16x8 *)(xs + (size_t)kb * 1536);
            const bf16x8 xm = *(const bf16x8 *)(xs + (size_t)kb * 1536 + 512);
            const bf16x8 xl = *(const bf16x8 *)(xs + (size_t)kb * 1536 + 1024);
            f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xh, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xm, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xl, c, 0, 0, 0);
            acc[0] = fmaf(half_to_float(sc.x & 0xffffu), c[0], acc[0]);
            acc[1] = fmaf(half_to_float(sc.x >> 16), c[1], acc[1]);
            acc[2] = fmaf(half_to_float(sc.y & 0xffffu), c[2], acc[2]);
            acc[3] = fmaf(half_to_float(sc.y >> 16), c[3], acc[3]);
        }
    } else {
        const uint16_t *wb = (const uint16_t *)a.w + (size_t)tile * kbn * 512 + lane * 8;
        for (int kb = kb_begin; kb < kb_end; kb++) {
            const bf16x8 wa = *(const bf16x8 *)(wb + (size_t)kb * 512);
            const bf16x8 xh = *(const bf16x8 *)(xs + (size_t)kb * 1536);
            const bf16x8 xm = *(const bf16x8 *)(xs + (size_t)kb * 1536 + 512);
            const bf16x8 xl = *(const bf16x8 *)(xs + (size_t)kb * 1536 + 1024);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xm, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xl, acc, 0, 0, 0);
        }
    }

    __shared__ f32x4 partial[4][64];
    partial[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;  // no barrier follows
    f32x4 v = partial[0][lane];
#pragma unroll
    for (int w = 1; w < 4; w++) {
        const f32x4 p = partial[w][lane];
        v[0] = __fadd_rn(v[0], p[0]);
        v[1] = __fadd_rn(v[1], p[1]);
        v[2] = __fadd_rn(v[2], p[2]);
        v[3] = __fadd_rn(v[3], p[3]);
    }

    // D fragment: lane holds rows row0 .. row0+3 of stream s.
    const int s = st * 16 + (lane & 15);
    const int row0 = tile * 16 + (lane >> 4) * 4;
    const bool live = s < a.streams;
    bool bad = false;
    if constexpr (EPI == EPI_STORE || EPI == EPI_RESIDUAL) {
        if (live) {
            float *o = a.out + (size_t)s * a.ld_out + row0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float y = v[r];
                if constexpr (EPI == EPI_STORE) {
                    if (a.bias) y = __fadd_rn(y, a.bias[row0 + r]);
                } else {
                    y = __fadd_rn(a.residual[(size_t)s * a.ld_out + row0 + r], y);
                }
                bad |= !isfinite(y);
                o[r] = y;
            }
        }
    } else if constexpr (EPI == EPI_GELU_SPLIT) {
        if (live) {
            float g[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                g[r] = gelu_erf(v[r]);
                bad |= !isfinite(g[r]);
            }
            store_split<4>(a.out_split, s, row0, a.out_kb, g);
        }
    } else {  // EPI_QKV: rows [0,512) q, [512,1024) k, [1024,1536) v
        if (live) {
            const int part = row0 >> 9, rr = row0 & 511;
            const int head = rr >> 6, d0 = rr & 63;
            int pos = a.positions[s];
            int block = 0;
            // Positions past the rope table or the block table, and block ids
            // outside the pool, are errors: flag them and write nothing.
            bool ok = pos >= 0 && pos < kMaxPositions && (pos >> 4) < a.table_stride;
            if (ok) {
                block = a.tables[(size_t)s * a.table_stride + (pos >> 4)];
                ok = (unsigned)block < a.blocks;
            }
            if (!ok) {
                atomicOr(a.status, 2);
                pos = 0;
            }
            float o[4] = {v[0], v[1], v[2], v[3]};
            if (part < 2) {
                // Interleaved pairs (d0, d0+1), (d0+2, d0+3): pair index d0/2.
                const float2 cs0 = a.rope[(size_t)pos * 32 + (d0 >> 1)];
                const float2 cs1 = a.rope[(size_t)pos * 32 + (d0 >> 1) + 1];
                o[0] = __fsub_rn(__fmul_rn(v[0], cs0.x), __fmul_rn(v[1], cs0.y));
                o[1] = __fadd_rn(__fmul_rn(v[0], cs0.y), __fmul_rn(v[1], cs0.x));
                o[2] = __fsub_rn(__fmul_rn(v[2], cs1.x), __fmul_rn(v[3], cs1.y));
                o[3] = __fadd_rn(__fmul_rn(v[2], cs1.y), __fmul_rn(v[3], cs1.x));
            }
#pragma unroll
            for (int r = 0; r < 4; r++) bad |= !isfinite(o[r]);
            if (part == 0) {
                // The 1/sqrt(64) score scale is a power of two: folding it
                // into q is exact.
                float4 qv = make_float4(o[0] * 0.125f, o[1] * 0.125f, o[2] * 0.125f,
                                        o[3] * 0.125f);
                *(float4 *)(a.q_out + (size_t)s * kWidth + rr) = qv;
            } else if (ok) {
                float *dst = a.kv + (size_t)a.layer * a.layer_stride +
                             ((size_t)block * kHeads + head) * 2048 + (part - 1) * 1024 +
                             (pos & 15) * 64 + d0;
                *(float4 *)dst = make_float4(o[0], o[1], o[2], o[3]);
            }
        }
    }
    flag_nonfinite(a.status, bad);
}

template <int EPI, bool Q8>
static int launch(const GemmArgs &a, hipStream_t stream) {
    if (a.n_rows <= 0 || a.n_rows % 16 || a.k_cols <= 0 || a.k_cols % 32 || a.streams <= 0)
        return bad_arguments("pgpu_gemm");
    dim3 grid(a.n_rows / 16, (a.streams + 15) / 16);
    hipLaunchKernelGGL((k_gemm<EPI, Q8>), grid, dim3(256), 0, stream, a);
    return launch_ok("pgpu_gemm");
}

static GemmArgs base_args(const pgpu_matrix *w, const uint16_t *xs, int streams, int *status) {
    GemmArgs a = {};
    a.xs = xs;
    a.w = w->values;
    a.wscale = w->scales;
    a.n_rows = (int)w->rows;
    a.k_cols = (int)w->columns;
    a.streams = streams;
    a.status = status;
    return a;
}

}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_gemm_store(void *stream, const pgpu_matrix *w, const uint16_t *xs,
                               int streams, const float *bias, float *out, int ld_out,
                               int *status) {
    GemmArgs a = base_args(w, xs, streams, status);
    a.out = out;
    a.ld_out = ld_out;
    a.bias = bias;
    return w->q8 ? launch<EPI_STORE, true>(a, (hipStream_t)stream)
                 : launch<EPI_STORE, false>(a, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_residual(void *stream, const pgpu_matrix *w, const uint16_t *xs,
                                  int streams, const float *residual, float *out, int *status) {
    GemmArgs a = base_args(w, xs, streams, status);
    a.out = out;
    a.ld_out = (int)w->rows;
    a.residual = residual;
    return w->q8 ? launch<EPI_RESIDUAL, true>(a, (hipStream_t)stream)
                 : launch<EPI_RESIDUAL, false>(a, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_gelu_split(void *stream, const pgpu_matrix *w, const uint16_t *xs,
                                    int streams, uint16_t *out_split, int *status) {
    GemmArgs a = base_args(w, xs, streams, status);
    a.out_split = out_split;
    a.out_kb = (int)w->rows / 32;
    return w->q8 ? launch<EPI_GELU_SPLIT, true>(a, (hipStream_t)stream)
                 : launch<EPI_GELU_SPLIT, false>(a, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_qkv(void *stream, const pgpu_matrix *w, const uint16_t *xs,
                             int streams, const pgpu_paged_kv *kv, int layer,
                             const int32_t *tables, int table_stride, const int32_t *positions,
                             const float *rope, float *q_out, int *status) {
    if (w->rows != 3 * kWidth || w->columns != kWidth || layer < 0 || layer >= kv->layers)
        return bad_arguments("pgpu_gemm_qkv");
    GemmArgs a = base_args(w, xs, streams, status);
    a.q_out = q_out;
    a.kv = kv->base;
    a.layer_stride = kv->layer_stride;
    a.blocks = (unsigned)kv->blocks;
    a.layer = layer;
    a.tables = tables;
    a.table_stride = table_stride;
    a.positions = positions;
    a.rope = (const float2 *)rope;
    return w->q8 ? launch<EPI_QKV, true>(a, (hipStream_t)stream)
                 : launch<EPI_QKV, false>(a, (hipStream_t)stream);
}
