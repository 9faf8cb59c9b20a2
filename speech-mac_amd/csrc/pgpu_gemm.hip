// Projection kernel of the decode step: Y[s][n] = sum_k X[s][k] * W[n][k]
// for B streams, on v_mfma_f32_16x16x32_bf16, with the producer of X fused
// in front and the consumer of Y fused behind.
//
// Replaces the fp32 SGEMM of phonon_linear (src/phonon_transformer.c:253-313)
// and the row dot of phonon_q8_matvec (src/phonon_q8.c:36-92); with its
// prologues/epilogues it also carries LayerNorm (:153-185), the attention
// output normalisation (:395-403), RoPE + KV append (:425-427), GELU
// (:202-216) and the residual adds (:440-451) of phonon_flow_layer_step.
//
// Operands
//   W  Q8_0: int8 values in MFMA A-fragment order, one 512-byte record per
//      (16-row tile, 32-column block); lane l holds row l%16, columns
//      8*(l/16) .. +7. The per-(row, block) fp16 scales sit in a separate
//      plane [tile][block][16]. Bytes per weight: 1 + 2/32 (same as Q8_0).
//   W  BF16: the same fragment order with bf16 values (1024-byte records).
//   X  split fragments (pgpu_common.hpp): three bf16 terms per activation,
//      read from global memory (SRC_SPLIT) or built in LDS by the prologue:
//      SRC_LN   LayerNorm of fp32 rows [streams][512];
//      SRC_ATTN merge of the split-attention partials (max, sum, acc).
// Arithmetic
//   Q8: per 32-column block, c = W_q8 . (X_hi + X_mid + X_lo) by three MFMAs
//   from zero (int8 and bf16 terms multiply exactly), then acc += scale*c,
//   i.e. the reference phonon_q8_dot order "sum += scale * partial".
//   BF16: the three MFMAs chain straight into the accumulator.
// Work decomposition (results never depend on scheduling): tasks of one
// 1024-thread work-group
//   SRC_SPLIT (gemm_split_task): 1 row tile x 16 streams; its 16 waves split
//   the column blocks into 16 ranges, summed in LDS in wave order.
//   SRC_LN / SRC_ATTN (gemm_wide_task, K = 512): 4 row tiles x 16 streams;
//   the prologue runs once with one wave per stream, then 16 waves take
//   (tile, quarter of the column blocks) pairs and the quarters are summed
//   in order. One prologue per 4 tiles, spread over 16 waves: the prologue,
//   not the MFMAs, is what the kernel's latency is made of.
#include <hip/hip_fp16.h>

#include "pgpu_attention.hpp"
#include "pgpu_common.hpp"
#include "phonon_gpu.h"

namespace pgpu {

enum Source { SRC_SPLIT = 0, SRC_LN = 1, SRC_ATTN = 2 };
enum Epilogue { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_GELU_SPLIT = 2, EPI_QKV = 3 };

struct GemmArgs {
    const uint16_t *xs;       // SRC_SPLIT: split fragments, k_cols/32 blocks per row
    const float *ln_x;        // SRC_LN: [streams][512] rows to normalise
    const float *ln_w, *ln_b; // SRC_LN: [512] affine
    float ln_eps;
    const float *part_acc;    // SRC_ATTN: [streams*8*max_splits][64]
    const float *part_ml;     // SRC_ATTN: [streams*8*max_splits][2]
    int max_splits;
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
    const int32_t *positions; // QKV and SRC_ATTN
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

// LDS operand buffer of the prologues: for column block kb, three 1 KB
// records (one per term) of 64 lanes x 8 bf16, in the MFMA B-operand order.
// Consecutive blocks are kLdsBlock elements apart: the 16-byte pad puts the
// 16 blocks one writer wave touches on distinct banks.
constexpr int kLdsBlock = 1536 + 8;

// Writes 8 activations of stream n (0..15 in the tile), columns
// [32kb + 8g, 32kb + 8g + 8), into the LDS operand buffer: one 16-byte
// record per split term.
__device__ inline void lds_store8(uint16_t *bsh, int n, int kb, int g, const float *v) {
    uint16_t h[8], m[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; i++) split3(v[i], h[i], m[i], l[i]);
    uint16_t *rec = bsh + kb * kLdsBlock + (g * 16 + n) * 8;
#pragma unroll
    for (int p = 0; p < 3; p++) {
        const uint16_t *src = p == 0 ? h : (p == 1 ? m : l);
        uint4 q;
        q.x = src[0] | (uint32_t)src[1] << 16;
        q.y = src[2] | (uint32_t)src[3] << 16;
        q.z = src[4] | (uint32_t)src[5] << 16;
        q.w = src[6] | (uint32_t)src[7] << 16;
        *(uint4 *)(rec + p * 512) = q;
    }
}

// Sum over the 64 lanes of a wave; every lane gets the same bits.
__device__ inline float wave_sum64(float v) {
    v = row16_sum(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// LayerNorm of 16 streams' 512-wide rows into LDS split fragments, by a
// 1024-thread work-group: wave n normalises stream n, lane j owns columns
// [8j, 8j+8). Two-pass fp32 moments; y = ((x - mean) * rstd) * w + b
// unfused, as the reference writes it (src/phonon_transformer.c:179-183).
__device__ inline bool prologue_ln(const GemmArgs &a, int st, uint16_t *bsh) {
    const int n = threadIdx.x >> 6, j = threadIdx.x & 63;
    const int s = st * 16 + n;
    const bool live = s < a.streams;  // uniform per wave
    float v[8];
    const float4 w0 = *(const float4 *)(a.ln_w + j * 8), w1 = *(const float4 *)(a.ln_w + j * 8 + 4);
    const float4 b0 = *(const float4 *)(a.ln_b + j * 8), b1 = *(const float4 *)(a.ln_b + j * 8 + 4);
    if (live) {
        const float4 x0 = *(const float4 *)(a.ln_x + (size_t)s * kWidth + j * 8);
        const float4 x1 = *(const float4 *)(a.ln_x + (size_t)s * kWidth + j * 8 + 4);
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.0f;
    }
    const float mean =
        wave_sum64(((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]))) *
        (1.0f / kWidth);
    float q2[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float c = __fsub_rn(v[i], mean);
        q2[i & 1] = fmaf(c, c, q2[i & 1]);
    }
    const float var = wave_sum64(q2[0] + q2[1]) * (1.0f / kWidth);
    const float rstd = 1.0f / sqrtf(var + a.ln_eps);
    const float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        v[i] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i], mean), rstd), ws[i]), bs[i]);
        bad |= !isfinite(v[i]);
        if (!live) v[i] = 0.0f;
    }
    lds_store8(bsh, n, j >> 2, j & 3, v);
    return bad && live;
}

// Merges the split-attention partials of 16 streams x 8 heads into LDS split
// fragments: out = sum_j acc_j e^(m_j - M) / sum_j l_j e^(m_j - M), M = max m_j
// (the normalisation after P.V of src/phonon_transformer.c:395-403), by a
// 1024-thread work-group: wave n merges stream n, lane (h = j/8, part = j%8)
// dims [8 part, 8 part + 8) of head h. Single pass in split order with a
// running maximum (accumulators rescaled when it grows), so every load of a
// group of 8 splits is issued at once: one memory round trip per 8 splits.
__device__ inline bool prologue_attn(const GemmArgs &a, int st, uint16_t *bsh) {
    const int n = threadIdx.x >> 6, j = threadIdx.x & 63;
    const int h = j >> 3, part = j & 7;
    const int s = st * 16 + n;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.0f;
    bool bad = false;
    if (s < a.streams) {
        const int count = a.positions[s] + 1;
        const int nsplit = min((count + kSplitKeys - 1) / kSplitKeys, a.max_splits);
        const size_t first = ((size_t)s * kHeads + h) * a.max_splits;
        const float2 *ml = (const float2 *)a.part_ml + first;
        float mx = -INFINITY, total = 0.0f;
        for (int j0 = 0; j0 < nsplit; j0 += 8) {
            float2 ml8[8];
            float4 acc[8][2];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int js = min(j0 + u, nsplit - 1);
                ml8[u] = ml[js];
                const float4 *src = (const float4 *)(a.part_acc + (first + js) * 64 + part * 8);
                acc[u][0] = src[0];
                acc[u][1] = src[1];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (j0 + u >= nsplit) break;
                const float m_new = fmaxf(mx, ml8[u].x);
                const float keep = expf(mx - m_new);  // 0 for the first split
                const float f = expf(ml8[u].x - m_new);
                mx = m_new;
                total = fmaf(ml8[u].y, f, total * keep);
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    v[4 * i] = fmaf(acc[u][i].x, f, v[4 * i] * keep);
                    v[4 * i + 1] = fmaf(acc[u][i].y, f, v[4 * i + 1] * keep);
                    v[4 * i + 2] = fmaf(acc[u][i].z, f, v[4 * i + 2] * keep);
                    v[4 * i + 3] = fmaf(acc[u][i].w, f, v[4 * i + 3] * keep);
                }
            }
        }
        bad = !(total > 0.0f) || !isfinite(total);
        const float inv = 1.0f / total;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[i] *= inv;
            bad |= !isfinite(v[i]);
        }
        if (bad) {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.0f;
        }
    }
    // Column 64h + 8 part: block 2h + part/4, group part%4.
    lds_store8(bsh, n, 2 * h + (part >> 2), part & 3, v);
    return bad;
}

// One chunk of CH column blocks of this lane's weight fragments.
template <bool Q8, int CH>
struct WChunk;
template <int CH>
struct WChunk<true, CH> {
    uint2 raw[CH], sc[CH];
};
template <int CH>
struct WChunk<false, CH> {
    bf16x8 w[CH];
};

template <bool Q8, int CH>
__device__ inline void load_weights(WChunk<Q8, CH> &c, const GemmArgs &a, int tile, int kbn,
                                    int lane, int kb0, int kb_end) {
#pragma unroll
    for (int u = 0; u < CH; u++) {
        const size_t kb = (size_t)min(kb0 + u, kb_end - 1);
        if constexpr (Q8) {
            c.raw[u] = *(const uint2 *)((const int8_t *)a.w + ((size_t)tile * kbn + kb) * 512 +
                                        lane * 8);
            c.sc[u] = *(const uint2 *)(a.wscale + ((size_t)tile * kbn + kb) * 16 +
                                       (lane >> 4) * 4);
        } else {
            c.w[u] = *(const bf16x8 *)((const uint16_t *)a.w + ((size_t)tile * kbn + kb) * 512 +
                                       lane * 8);
        }
    }
}

// acc += W_chunk . X_chunk. No control flow between loads and MFMAs: a block
// past the wave's range contributes 0 (scale 0 / zero fragment).
template <bool Q8, int CH>
__device__ inline void mfma_chunk(f32x4 &acc, const WChunk<Q8, CH> &w, const bf16x8 *xh,
                                  const bf16x8 *xm, const bf16x8 *xl, int kb0, int kb_end) {
#pragma unroll
    for (int u = 0; u < CH; u++) {
        const bool used = kb0 + u < kb_end;
        if constexpr (Q8) {
            const bf16x8 wa = q8_to_bf16(w.raw[u]);
            f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xh[u], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xm[u], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xl[u], c, 0, 0, 0);
            const uint2 s = used ? w.sc[u] : make_uint2(0u, 0u);
            acc[0] = fmaf(half_to_float(s.x & 0xffffu), c[0], acc[0]);
            acc[1] = fmaf(half_to_float(s.x >> 16), c[1], acc[1]);
            acc[2] = fmaf(half_to_float(s.y & 0xffffu), c[2], acc[2]);
            acc[3] = fmaf(half_to_float(s.y >> 16), c[3], acc[3]);
        } else {
            const bf16x8 wa = used ? w.w[u] : bf16x8{};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xh[u], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xm[u], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xl[u], acc, 0, 0, 0);
        }
    }
}

// Operands of the epilogue of one lane (rows row0..row0+3 of stream s).
struct EpiOperands {
    float4 add;          // STORE: bias, RESIDUAL: residual
    bool has_add;
    float2 cs0, cs1;     // QKV: (cos, sin) of the lane's two RoPE pairs
    int pos, block;      // QKV: append position and its pool block
    bool ok;             // QKV: position and block are valid
};

template <int EPI>
__device__ inline void load_epilogue(EpiOperands &e, const GemmArgs &a, int s, int row0,
                                     bool live) {
    e.add = make_float4(0.f, 0.f, 0.f, 0.f);
    e.has_add = false;
    if (!live) return;
    if constexpr (EPI == EPI_STORE) {
        if (a.bias) {
            e.add = *(const float4 *)(a.bias + row0);
            e.has_add = true;
        }
    } else if constexpr (EPI == EPI_RESIDUAL) {
        e.add = *(const float4 *)(a.residual + (size_t)s * a.ld_out + row0);
        e.has_add = true;
    } else if constexpr (EPI == EPI_QKV) {
        // Positions past the rope table or the block table, and block ids
        // outside the pool, are errors: flagged, and nothing is written.
        int pos = a.positions[s];
        e.ok = pos >= 0 && pos < kMaxPositions && (pos >> 4) < a.table_stride;
        e.block = 0;
        if (e.ok) {
            e.block = a.tables[(size_t)s * a.table_stride + (pos >> 4)];
            e.ok = (unsigned)e.block < a.blocks;
        }
        if (!e.ok) pos = 0;
        e.pos = pos;
        const int d0 = (row0 & 511) & 63;
        e.cs0 = a.rope[(size_t)pos * 32 + (d0 >> 1)];
        e.cs1 = a.rope[(size_t)pos * 32 + (d0 >> 1) + 1];
    }
}

// Consumer of one lane's four results v (rows row0..row0+3 of stream s).
// Returns true if a non-finite value was produced.
template <int EPI>
__device__ inline bool epilogue(const GemmArgs &a, const EpiOperands &e, const f32x4 &v, int s,
                                int row0, bool live) {
    bool bad = false;
    if constexpr (EPI == EPI_STORE || EPI == EPI_RESIDUAL) {
        if (live) {
            float *o = a.out + (size_t)s * a.ld_out + row0;
            const float add[4] = {e.add.x, e.add.y, e.add.z, e.add.w};
            float y[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // bias + dot (STORE) or residual + dot (RESIDUAL); 0 + dot
                // without a bias is exact.
                y[r] = EPI == EPI_STORE ? (e.has_add ? __fadd_rn(v[r], add[r]) : v[r])
                                        : __fadd_rn(add[r], v[r]);
                bad |= !isfinite(y[r]);
            }
            *(float4 *)o = make_float4(y[0], y[1], y[2], y[3]);
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
            const bool ok = e.ok;
            const int pos = e.pos, block = e.block;
            if (!ok) atomicOr(a.status, 2);
            float o[4] = {v[0], v[1], v[2], v[3]};
            if (part < 2) {
                // Interleaved pairs (d0, d0+1), (d0+2, d0+3): pair index d0/2.
                const float2 cs0 = e.cs0, cs1 = e.cs1;
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
    return bad;
}

// Tasks: the unit of work of one 1024-thread work-group, run by the
// single-phase kernels below (one task per work-group) and by the decode
// layer kernel (several tasks per work-group, phase after phase), so both
// produce the same bits.

// LDS of a task: the prologue's operand buffer, reused for partial sums.
constexpr int kTaskLds = 16 * kLdsBlock;

// Split-fragment rows from global memory (any K): one row tile x 16
// streams. The 16 waves split the column blocks into 16 contiguous ranges
// (4 blocks each at K = 2048, all requested at once; chunks of CH, the next
// chunk's weights requested before the current chunk's MFMAs), summed in
// LDS in wave order.
template <int EPI, bool Q8, int CH>
__device__ inline void gemm_split_task(const GemmArgs &a, int tile, int st, uint16_t *lds) {
    constexpr int NW = 16;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int kbn = a.k_cols >> 5;
    const int per = (kbn + NW - 1) / NW;
    const int kb_begin = wave * per;
    const int kb_end = min(kbn, kb_begin + per);

    // D fragment of this lane: rows row0 .. row0+3 of stream s.
    const int s = st * 16 + (lane & 15);
    const int row0 = tile * 16 + (lane >> 4) * 4;
    const bool live = s < a.streams;

    WChunk<Q8, CH> w;
    if (kb_begin < kb_end) load_weights(w, a, tile, kbn, lane, kb_begin, kb_end);
    EpiOperands e;
    if (wave == 0) load_epilogue<EPI>(e, a, s, row0, live);

    const uint16_t *xs = a.xs + (size_t)st * kbn * 1536 + lane * 8;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb0 = kb_begin; kb0 < kb_end; kb0 += CH) {
        bf16x8 xh[CH], xm[CH], xl[CH];
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const size_t kb = (size_t)min(kb0 + u, kb_end - 1) * 1536;
            xh[u] = *(const bf16x8 *)(xs + kb);
            xm[u] = *(const bf16x8 *)(xs + kb + 512);
            xl[u] = *(const bf16x8 *)(xs + kb + 1024);
        }
        WChunk<Q8, CH> next;
        if (kb0 + CH < kb_end) load_weights(next, a, tile, kbn, lane, kb0 + CH, kb_end);
        mfma_chunk(acc, w, xh, xm, xl, kb0, kb_end);
        w = next;
    }

    f32x4 *partial = (f32x4 *)lds;
    __syncthreads();  // the buffer may still be read by a previous task
    partial[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4 v = acc;
#pragma unroll
    for (int w2 = 1; w2 < NW; w2++) {
        const f32x4 p = partial[w2 * 64 + lane];
        v[0] = __fadd_rn(v[0], p[0]);
        v[1] = __fadd_rn(v[1], p[1]);
        v[2] = __fadd_rn(v[2], p[2]);
        v[3] = __fadd_rn(v[3], p[3]);
    }
    flag_nonfinite(a.status, epilogue<EPI>(a, e, v, s, row0, live));
}

// Operand built by a prologue (LayerNorm or the attention merge; K = 512):
// 4 row tiles x 16 streams. The prologue runs once per 64 rows with 8
// values per lane (one wave per stream); wave w = 4q + t then computes
// column blocks [4q, 4q+4) of tile t, and the 4 quarters of a tile are
// added in order. The wave's weights and the epilogue operands are
// requested before the prologue, so their latency overlaps it.
template <int SRC, int EPI, bool Q8>
__device__ inline void gemm_wide_task(const GemmArgs &a, int bx, int st, uint16_t *bsh) {
    constexpr int kbn = kWidth / 32, KBW = kbn / 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t = wave & 3, q = wave >> 2;
    const int tile = bx * 4 + t;
    const bool active = tile < (a.n_rows >> 4);  // uniform per wave
    const int kb0 = q * KBW;
    const int s = st * 16 + (lane & 15);
    const bool live = s < a.streams;
    const int row0 = tile * 16 + (lane >> 4) * 4;

    WChunk<Q8, KBW> w;
    if (active) load_weights(w, a, tile, kbn, lane, kb0, kb0 + KBW);
    EpiOperands e;
    if (active && q == 0) load_epilogue<EPI>(e, a, s, row0, live);

    __syncthreads();  // the buffer may still be read by a previous task
    const bool bad_in = SRC == SRC_LN ? prologue_ln(a, st, bsh) : prologue_attn(a, st, bsh);
    flag_nonfinite(a.status, bad_in);
    __syncthreads();

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (active) {
        bf16x8 xh[KBW], xm[KBW], xl[KBW];
        const uint16_t *xs = bsh + kb0 * kLdsBlock + lane * 8;
#pragma unroll
        for (int u = 0; u < KBW; u++) {
            xh[u] = *(const bf16x8 *)(xs + u * kLdsBlock);
            xm[u] = *(const bf16x8 *)(xs + u * kLdsBlock + 512);
            xl[u] = *(const bf16x8 *)(xs + u * kLdsBlock + 1024);
        }
        mfma_chunk(acc, w, xh, xm, xl, kb0, kb0 + KBW);
    }
    // Quarter sums through LDS (the operand buffer is free once every wave
    // has its B operands): partial[q][t].
    __syncthreads();
    f32x4 *partial = (f32x4 *)bsh;
    partial[wave * 64 + lane] = acc;
    __syncthreads();
    if (q != 0 || !active) return;
    f32x4 v = acc;
#pragma unroll
    for (int q2 = 1; q2 < 4; q2++) {
        const f32x4 p = partial[(q2 * 4 + t) * 64 + lane];
        v[0] = __fadd_rn(v[0], p[0]);
        v[1] = __fadd_rn(v[1], p[1]);
        v[2] = __fadd_rn(v[2], p[2]);
        v[3] = __fadd_rn(v[3], p[3]);
    }
    flag_nonfinite(a.status, epilogue<EPI>(a, e, v, s, row0, live));
}

template <int EPI, bool Q8, int CH>
__global__ __launch_bounds__(1024) void k_gemm(GemmArgs a) {
    __shared__ uint16_t lds[16 * 64 * 8];  // 16 waves x 64 lanes x f32x4
    gemm_split_task<EPI, Q8, CH>(a, blockIdx.x, blockIdx.y, lds);
}

template <int SRC, int EPI, bool Q8>
__global__ __launch_bounds__(1024) void k_gemm_wide(GemmArgs a) {
    __shared__ uint16_t bsh[kTaskLds];
    gemm_wide_task<SRC, EPI, Q8>(a, blockIdx.x, blockIdx.y, bsh);
}

// ---------------------------------------------------------------------
// Paired decode kernel: one launch holds the split attention of one stream
// group (layer l) and the projection chain of another group that follows
// its own attention: out projection, MLP in, MLP out and the next layer's
// QKV (src/phonon_transformer.c:437-451, 418-427). The attention is HBM
// bound and the projections are latency chains, so running them side by
// side hides the chain. Work-groups [0, chain_wgs) run the chain, phase
// after phase, with a device-wide barrier between phases; they hold the
// lowest block ids, so all of them are resident before any attention
// work-group starts. The rest run two attention split units each. Every
// task is the code of the single-phase kernels, so results are bit-identical
// to running the phases one launch at a time.

enum ChainPhase { PH_OUT = 0, PH_MLP_IN = 1, PH_MLP_OUT = 2, PH_QKV = 3 };

struct PairArgs {
    AttnArgs att;           // attention of streams [att_stream0, +att_streams)
    int att_stream0, att_units;  // units = 8 heads x att.max_splits x streams
    GemmArgs chain[4];      // ChainPhase order, for stream tiles [st0, st0 + tiles)
    int phases;             // 0, 3 (last layer) or 4
    int st0, tiles, chain_wgs;
    unsigned *counter;      // zero at launch; one per launch
    int *status;
};

// Device-wide barrier among the chain's work-groups: release, count, wait,
// acquire. The wait is bounded: a work-group that waits too long flags
// status bit 4 (results are then unspecified) and goes on, so the kernel
// always ends.
__device__ inline void chain_barrier(unsigned *counter, unsigned target, int *status) {
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        atomicAdd(counter, 1u);
        int spins = 0;
        while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++spins > (1 << 20)) {
                atomicOr(status, 4);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        __threadfence();
    }
    __syncthreads();
}

template <bool Q8>
__global__ __launch_bounds__(1024) void k_decode_pair(PairArgs p) {
    __shared__ uint4 lds4[kTaskLds / 8];
    uint16_t *lds = (uint16_t *)lds4;
    if ((int)blockIdx.x < p.chain_wgs) {
        for (int ph = 0; ph < p.phases; ph++) {
            if (ph > 0) chain_barrier(p.counter, (unsigned)(p.chain_wgs * ph), p.status);
            const GemmArgs &a = p.chain[ph];
            const int nx = ph == PH_MLP_OUT ? a.n_rows / 16 : (a.n_rows / 16 + 3) / 4;
            const int tasks = nx * p.tiles;
            for (int task = blockIdx.x; task < tasks; task += p.chain_wgs) {
                const int bx = task % nx, st = p.st0 + task / nx;
                if (ph == PH_OUT)
                    gemm_wide_task<SRC_ATTN, EPI_RESIDUAL, Q8>(a, bx, st, lds);
                else if (ph == PH_MLP_IN)
                    gemm_wide_task<SRC_LN, EPI_GELU_SPLIT, Q8>(a, bx, st, lds);
                else if (ph == PH_MLP_OUT)
                    gemm_split_task<EPI_RESIDUAL, Q8, 4>(a, bx, st, lds);
                else
                    gemm_wide_task<SRC_LN, EPI_QKV, Q8>(a, bx, st, lds);
            }
        }
        return;
    }
    // Attention: units (head fastest, then split, then stream), two per
    // work-group (waves 0-7 and 8-15).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int u = ((int)blockIdx.x - p.chain_wgs) * 2 + (wave >> 3);
    const bool exists = u < p.att_units;
    const int head = u & 7, rest = u >> 3;
    const int split = rest % p.att.max_splits;
    const int s = p.att_stream0 + (exists ? rest / p.att.max_splits : 0);
    AttnShared *sh = (AttnShared *)lds4;
    attend_split(p.att, head, split, s, wave & 7, sh[wave >> 3], exists);
}

template <int SRC, int EPI, bool Q8>
static int launch(const GemmArgs &a, hipStream_t stream) {
    if (a.n_rows <= 0 || a.n_rows % 16 || a.k_cols <= 0 || a.k_cols % 32 || a.streams <= 0 ||
        (SRC != SRC_SPLIT && a.k_cols != kWidth))
        return bad_arguments("pgpu_gemm");
    if constexpr (SRC != SRC_SPLIT) {
        const dim3 grid((a.n_rows / 16 + 3) / 4, (a.streams + 15) / 16);
        hipLaunchKernelGGL((k_gemm_wide<SRC, EPI, Q8>), grid, dim3(1024), 0, stream, a);
    } else {
        const dim3 grid(a.n_rows / 16, (a.streams + 15) / 16);
        hipLaunchKernelGGL((k_gemm<EPI, Q8, 4>), grid, dim3(1024), 0, stream, a);
    }
    return launch_ok("pgpu_gemm");
}

template <int EPI>
static int dispatch(const GemmArgs &a, int q8, hipStream_t stream) {
    const int src = a.ln_x ? SRC_LN : (a.part_acc ? SRC_ATTN : SRC_SPLIT);
    if (src == SRC_LN)
        return q8 ? launch<SRC_LN, EPI, true>(a, stream) : launch<SRC_LN, EPI, false>(a, stream);
    if (src == SRC_ATTN)
        return q8 ? launch<SRC_ATTN, EPI, true>(a, stream)
                  : launch<SRC_ATTN, EPI, false>(a, stream);
    return q8 ? launch<SRC_SPLIT, EPI, true>(a, stream)
              : launch<SRC_SPLIT, EPI, false>(a, stream);
}

// Fills the operand-source fields from a pgpu_gemm_input.
static bool set_input(GemmArgs &a, const pgpu_gemm_input *in) {
    if (!in) return false;
    const int kinds = (in->split != nullptr) + (in->ln_rows != nullptr) +
                      (in->attn_acc != nullptr);
    if (kinds != 1) return false;
    a.xs = in->split;
    a.ln_x = in->ln_rows;
    a.ln_w = in->ln_weight;
    a.ln_b = in->ln_bias;
    a.ln_eps = in->ln_epsilon;
    a.part_acc = in->attn_acc;
    a.part_ml = in->attn_ml;
    a.max_splits = in->attn_max_splits;
    if (a.ln_x && (!a.ln_w || !a.ln_b)) return false;
    if (a.part_acc && (!a.part_ml || a.max_splits <= 0 || !in->attn_positions)) return false;
    if (a.part_acc) a.positions = in->attn_positions;
    return true;
}

static bool base_args(GemmArgs &a, const pgpu_matrix *w, const pgpu_gemm_input *in, int streams,
                      int *status) {
    a = GemmArgs{};
    a.w = w->values;
    a.wscale = w->scales;
    a.n_rows = (int)w->rows;
    a.k_cols = (int)w->columns;
    a.streams = streams;
    a.status = status;
    return set_input(a, in);
}

}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_gemm_store(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *in,
                               int streams, const float *bias, float *out, int ld_out,
                               int *status) {
    GemmArgs a;
    if (!base_args(a, w, in, streams, status)) return bad_arguments("pgpu_gemm_store");
    a.out = out;
    a.ld_out = ld_out;
    a.bias = bias;
    return dispatch<EPI_STORE>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_residual(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *in,
                                  int streams, const float *residual, float *out, int *status) {
    GemmArgs a;
    if (!base_args(a, w, in, streams, status)) return bad_arguments("pgpu_gemm_residual");
    a.out = out;
    a.ld_out = (int)w->rows;
    a.residual = residual;
    return dispatch<EPI_RESIDUAL>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_gelu_split(void *stream, const pgpu_matrix *w,
                                    const pgpu_gemm_input *in, int streams, uint16_t *out_split,
                                    int *status) {
    GemmArgs a;
    if (!base_args(a, w, in, streams, status)) return bad_arguments("pgpu_gemm_gelu_split");
    a.out_split = out_split;
    a.out_kb = (int)w->rows / 32;
    return dispatch<EPI_GELU_SPLIT>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_qkv(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *in,
                             int streams, const pgpu_paged_kv *kv, int layer,
                             const int32_t *tables, int table_stride, const int32_t *positions,
                             const float *rope, float *q_out, int *status) {
    GemmArgs a;
    if (w->rows != 3 * kWidth || w->columns != kWidth || layer < 0 || layer >= kv->layers ||
        !base_args(a, w, in, streams, status) || a.part_acc)
        return bad_arguments("pgpu_gemm_qkv");
    a.q_out = q_out;
    a.kv = kv->base;
    a.layer_stride = kv->layer_stride;
    a.blocks = (unsigned)kv->blocks;
    a.layer = layer;
    a.tables = tables;
    a.table_stride = table_stride;
    a.positions = positions;
    a.rope = (const float2 *)rope;
    return dispatch<EPI_QKV>(a, w->q8, (hipStream_t)stream);
}

static bool chain_phase_args(GemmArgs &a, const pgpu_matrix *w, const pgpu_gemm_input &in,
                             int streams, int *status) {
    return w && w->values && (!w->q8 || w->scales) && base_args(a, w, &in, streams, status) &&
           a.n_rows > 0 && a.n_rows % 16 == 0 && a.k_cols > 0 && a.k_cols % 32 == 0;
}

extern "C" int pgpu_decode_pair(void *stream, const pgpu_pair_attention *att,
                                const pgpu_pair_chain *ch, const pgpu_paged_kv *kv,
                                int table_stride, const float *rope, unsigned *counter,
                                int *status) {
    if ((!att && !ch) || !kv || !status || table_stride <= 0 || (ch && (!counter || !rope)))
        return bad_arguments("pgpu_decode_pair");
    PairArgs p{};
    p.status = status;
    p.counter = counter;
    int q8 = -1;
    if (att) {
        const pgpu_attention_scratch &sc = att->scratch;
        if (!att->q || !att->tables || !att->positions || att->streams <= 0 ||
            att->layer < 0 || att->layer >= kv->layers || sc.max_splits <= 0 ||
            att->streams > sc.max_streams)
            return bad_arguments("pgpu_decode_pair");
        AttnArgs &a = p.att;
        a.q = att->q;
        a.kv = kv->base;
        a.layer_stride = kv->layer_stride;
        a.blocks = (unsigned)kv->blocks;
        a.layer = att->layer;
        a.tables = att->tables;
        a.table_stride = table_stride;
        a.positions = att->positions;
        a.streams = att->streams;
        a.max_splits = sc.max_splits;
        a.part_acc = sc.part_acc;
        a.part_ml = sc.part_ml;
        a.status = status;
        p.att_units = kHeads * sc.max_splits * att->streams;
    }
    if (ch) {
        const int n = ch->streams;
        if (n <= 0 || ch->layer < 0 || ch->layer >= kv->layers ||
            (ch->qkv_next && ch->layer + 1 >= kv->layers) || !ch->out || !ch->mlp_in ||
            !ch->mlp_out || ch->out->rows != (size_t)kWidth || ch->mlp_in->columns != (size_t)kWidth ||
            ch->mlp_out->rows != (size_t)kWidth || ch->mlp_out->columns != ch->mlp_in->rows ||
            ch->scratch.max_splits <= 0 || n > ch->scratch.max_streams)
            return bad_arguments("pgpu_decode_pair");
        q8 = ch->out->q8;
        if (ch->mlp_in->q8 != q8 || ch->mlp_out->q8 != q8 || (ch->qkv_next && ch->qkv_next->q8 != q8))
            return bad_arguments("pgpu_decode_pair");
        pgpu_gemm_input in{};
        in.attn_acc = ch->scratch.part_acc;
        in.attn_ml = ch->scratch.part_ml;
        in.attn_positions = ch->positions;
        in.attn_max_splits = ch->scratch.max_splits;
        GemmArgs &o = p.chain[PH_OUT];
        if (!chain_phase_args(o, ch->out, in, n, status)) return bad_arguments("pgpu_decode_pair");
        o.out = ch->r;
        o.ld_out = kWidth;
        o.residual = ch->input;
        in = pgpu_gemm_input{};
        in.ln_rows = ch->r;
        in.ln_weight = ch->norm2_weight;
        in.ln_bias = ch->norm2_bias;
        in.ln_epsilon = ch->ln_epsilon;
        GemmArgs &mi = p.chain[PH_MLP_IN];
        if (!chain_phase_args(mi, ch->mlp_in, in, n, status) || mi.k_cols != kWidth)
            return bad_arguments("pgpu_decode_pair");
        mi.out_split = ch->hidden;
        mi.out_kb = mi.n_rows / 32;
        in = pgpu_gemm_input{};
        in.split = ch->hidden;
        GemmArgs &mo = p.chain[PH_MLP_OUT];
        if (!chain_phase_args(mo, ch->mlp_out, in, n, status))
            return bad_arguments("pgpu_decode_pair");
        mo.out = ch->output;
        mo.ld_out = kWidth;
        mo.residual = ch->r;
        p.phases = 3;
        if (ch->qkv_next) {
            in = pgpu_gemm_input{};
            in.ln_rows = ch->output;
            in.ln_weight = ch->norm1_next_weight;
            in.ln_bias = ch->norm1_next_bias;
            in.ln_epsilon = ch->ln_epsilon;
            GemmArgs &q = p.chain[PH_QKV];
            if (ch->qkv_next->rows != 3 * (size_t)kWidth ||
                !chain_phase_args(q, ch->qkv_next, in, n, status) || q.k_cols != kWidth)
                return bad_arguments("pgpu_decode_pair");
            q.q_out = ch->q_next;
            q.kv = kv->base;
            q.layer_stride = kv->layer_stride;
            q.blocks = (unsigned)kv->blocks;
            q.layer = ch->layer + 1;
            q.tables = ch->tables;
            q.table_stride = table_stride;
            q.positions = ch->positions;
            q.rope = (const float2 *)rope;
            p.phases = 4;
        }
        p.st0 = 0;
        p.tiles = (n + 15) / 16;
        // One round of tasks per phase (the widest phase has 32 tasks per
        // tile), at most 64 chain work-groups.
        p.chain_wgs = min(64, 32 * p.tiles);
    }
    const int grid = p.chain_wgs + (p.att_units + 1) / 2;
    if (q8 == 0)
        hipLaunchKernelGGL(k_decode_pair<false>, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
    else
        hipLaunchKernelGGL(k_decode_pair<true>, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
    return launch_ok("pgpu_decode_pair");
}
