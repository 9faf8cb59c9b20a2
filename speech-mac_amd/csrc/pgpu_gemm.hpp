// Projection tasks of the decode step: Y[s][n] = sum_k X[s][k] * W[n][k] for
// one 16-stream tile, on v_mfma_f32_16x16x32_bf16, with the producer of X
// fused in front (prologue) and the consumer of Y behind (epilogue).
//
// A task is the work of one 512-thread (8-wave) work-group. The same task
// code runs in the single-phase kernels (pgpu_gemm.hip, one task per
// work-group) and in the one-launch decode step (pgpu_flow.hip, where a
// task first waits for the tasks it depends on), so both produce the same
// bits.
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
//      read from global memory (SRC_SPLIT) or built in LDS by a prologue:
//      SRC_LN   LayerNorm of fp32 rows [streams][512];
//      SRC_ROWS fp32 rows [streams][512] as they are;
//      SRC_ATTN merge of the split-attention partials (max, sum, acc);
//      SRC_LN_MOD LayerNorm (optional affine) then adaLN modulation
//               h * (1 + scale) + shift by per-stream rows (flow head);
//      SRC_SPLIT_LDS split fragments from global memory copied into LDS
//               once per work-group (a K = 512 projection of many rows).
// Arithmetic
//   Q8: per 32-column block, c = W_q8 . (X_hi + X_mid + X_lo) by three MFMAs
//   from zero (int8 and bf16 terms multiply exactly), then acc += scale*c,
//   i.e. the reference phonon_q8_dot order "sum += scale * partial".
//   BF16: the three MFMAs chain straight into the accumulator.
// q and appended K/V are stored device-scope write-through (sc1), and the
// other outputs too when GemmArgs::wt_out is set, so a task on another XCD
// that waits for this one reads them from memory; see pgpu_flow.hip.
#pragma once

#include <hip/hip_fp16.h>

#include "pgpu_common.hpp"
#include "phonon_gpu.h"

namespace pgpu {

enum Source {
    SRC_SPLIT = 0,
    SRC_LN = 1,
    SRC_ATTN = 2,
    SRC_ROWS = 3,
    SRC_LN_MOD = 4,
    SRC_SPLIT_LDS = 5,
    SRC_ATTN_TAGGED = 6,  // merge of tagged split partials, polled (one-launch step)
    SRC_LN_PARTS = 7,     // LayerNorm of r + the fused MLP's partials, polled (one-launch step)
    SRC_LN_MOD_PARTS = 8, // SRC_LN_MOD of x_prev + gate * (the partials' sum + bias) (head chain)
};
enum Epilogue {
    EPI_STORE = 0,
    EPI_RESIDUAL = 1,
    EPI_GELU_SPLIT = 2,
    EPI_QKV = 3,
    EPI_SILU_SPLIT = 4,  // split fragments of SiLU((dot + bias) + bias2)
    EPI_GATED = 5,       // residual + gate * (dot + bias); optionally also split fragments
    EPI_GELU_W2 = 6,     // GELU, then times the task's 64 columns of W2: a partial
    EPI_SILU_W2 = 7,     // SiLU(dot + bias), then times the task's 64 columns of W2: a partial
};

constexpr int kTaskWaves = 8, kTaskThreads = 64 * kTaskWaves;

// ---------------------------------------------------------------------------
// Tagged hand-off words (one-launch step). A value handed from one task to
// another is a 64-bit word: its fp32 bits in the low half and the tag of
// the step that produced it in the high half, written by one 64-bit
// device-scope store. The consumer loads the words themselves with
// device-scope loads until every tag is the current step's: a word that
// carries the tag carries its value, so the producer neither drains its
// stores nor counts itself done, and the consumer needs no counter. Every
// such word has its own address per layer and is written at most once per
// step, so a stale word carries an older tag.
struct TagPoll {
    uint32_t tag;
    int *status;      // bit 4: some wait gave up; every poll then stops
    uint64_t ticks;   // give-up bound on the 100 MHz constant clock
    // The first load is a plain one (cacheable in the XCD's L2, so the
    // tasks of an XCD that read the same words share one fetch): for a
    // consumer that first waited for its producers' count. Words whose tag
    // it does not find are then polled at device scope.
    bool plain_first;
};

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

// Buffer resource of `bytes` bytes from `base`; both must be the same in
// every lane of the wave (they are read from the first active lane, so the
// resource lives in scalar registers).
__device__ inline __amdgpu_buffer_rsrc_t tag_rsrc(const void *base, uint32_t bytes) {
    const uint64_t p = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)((uint64_t)hi << 32 | lo), 0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Two consecutive words at byte offset `off`: one 16-byte load at device
// scope (sc1), so it is served coherently across the XCDs' L2s; or, with
// `plain`, a cacheable load.
__device__ inline u32x4 tag_load2(__amdgpu_buffer_rsrc_t r, uint32_t off, bool plain = false) {
    return plain ? __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0)
                 : __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}

__device__ inline bool tag_ok2(const u32x4 &w, uint32_t tag) {
    return w.y == tag && w.w == tag;
}

// Between two polls of a wave: true (and the status bit set) once the wave
// has polled longer than the bound, or another wait gave up.
__device__ inline bool tag_give_up(const TagPoll &tp, uint64_t t0, int round) {
    bool stop = wall_clock64() - t0 > tp.ticks;
    if ((round & 7) == 7)
        stop |= (__hip_atomic_load(tp.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 4) != 0;
    if (stop && (threadIdx.x & 63) == 0) atomicOr(tp.status, 4);
    return stop;
}

__device__ inline void store_tagged(uint64_t *p, float v, uint32_t tag) {
    __hip_atomic_store(p, (uint64_t)fbits(v) | (uint64_t)tag << 32, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline void store_tagged4(uint64_t *p, float4 v, uint32_t tag) {
    store_tagged(p, v.x, tag);
    store_tagged(p + 1, v.y, tag);
    store_tagged(p + 2, v.z, tag);
    store_tagged(p + 3, v.w, tag);
}

// Four consecutive tagged values at byte offset `off` of r, for a lane that
// needs them (`live`; the others get zeros), polled until all carry the
// tag. Every lane of the wave must call it.
__device__ inline float4 poll_tagged4(__amdgpu_buffer_rsrc_t r, uint32_t off, bool live,
                                      const TagPoll &tp) {
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    const uint64_t t0 = wall_clock64();
    for (int round = 0;; round++) {
        // Each round loads again: nothing may be hoisted out of the loop.
        __asm__ volatile("" ::: "memory");
        if (live) {
            const bool plain = round == 0 && tp.plain_first;
            a = tag_load2(r, off, plain);
            b = tag_load2(r, off + 16, plain);
        }
        if (__all(!live || (tag_ok2(a, tp.tag) && tag_ok2(b, tp.tag)))) break;
        if (tag_give_up(tp, t0, round)) break;
        __builtin_amdgcn_s_sleep(1);
    }
    return make_float4(bitsf(a.x), bitsf(a.z), bitsf(b.x), bitsf(b.z));
}

struct GemmArgs {
    const uint16_t *xs;       // SRC_SPLIT: split fragments, k_cols/32 blocks per row
    const float *ln_x;        // SRC_LN / SRC_ROWS: [streams][512] rows
    const float *ln_w, *ln_b; // SRC_LN: [512] affine
    float ln_eps;
    const float *part_acc;    // SRC_ATTN: [streams*8*max_splits][64]
    const float *part_ml;     // SRC_ATTN: [streams*8*max_splits][2]
    int max_splits;
    const void *w;            // weight fragments
    const uint16_t *wscale;   // Q8 only
    const float *wscale_f;    // prefill projections: fp32 scales of bf16 fragments, or null
    int n_rows, k_cols, streams;
    float *out;               // STORE / RESIDUAL: [streams][ld_out]
    int ld_out;
    const float *bias;        // STORE: optional [n_rows]
    const float *residual;    // RESIDUAL: [streams][ld_out]
    uint16_t *out_split;      // GELU_SPLIT: split fragments with out_kb blocks per row
    int out_kb;
    int out_terms;            // GELU_SPLIT: split terms written (0: all three)
    float *q_out;             // QKV: [streams][512]
    float *kv;                // QKV: paged pool base
    size_t layer_stride;      // floats per layer of the pool
    unsigned blocks;          // QKV: blocks per layer of the pool
    int layer;
    const int32_t *tables;
    int table_stride;
    const int32_t *positions; // QKV and SRC_ATTN: positions[s] + pos_delta
    int pos_delta = 0;        // steps the stored positions trail the step's
    const float2 *rope;       // [8192][32] (cos, sin)
    int *status;
    bool wt_out;              // STORE / RESIDUAL / GELU_SPLIT outputs write-through
    const float *bias2;       // SILU_SPLIT: optional second [n_rows] vector
    const float *gate;        // GATED: [streams][ld_gate] rows (columns [0, n_rows))
    int ld_gate;
    const float *mod;         // SRC_LN_MOD: shift row at mod + s * ld_mod, scale at +512
    int ld_mod;
    bool plain_rows;          // single-phase launch: ln_x rows are used as they are
    bool plain_qkv;           // QKV: q and K/V stored plainly (read only by later launches)
    int split_terms;          // prefill projections: split terms of X used (2 or 3)
    // Tagged hand-off rows of the one-launch step (null: the plain operands
    // above): tx replaces ln_x, tres replaces residual, tout replaces out,
    // each [tile][16][512] words (see TagPoll); ready_mark (optional)
    // receives the time the polled inputs were all seen.
    const uint64_t *tx, *tres;
    uint64_t *tout;
    TagPoll tp;
    // SRC_ATTN_TAGGED: the layer's tagged split partials,
    // [tiles*16][8][max_splits][PGPU_FLOW_PART_WORDS] (P.V [64], max, sum).
    const uint64_t *tparts;
    // QKV (optional): q (scaled), k and v also as tagged words, part p at
    // tqkv + p * tqkv_part, [tiles*16][512] each.
    uint64_t *tqkv;
    size_t tqkv_part;
    uint64_t *ready_mark;
    // Fused MLP (one-launch step, PGPU_FLOW_HANDOFF_FUSED_MLP):
    // SRC_LN_PARTS: x = r + sum of the PGPU_FLOW_MLP_IN_TASKS partials at
    // tmlp ([task][mlp_streams][512] fp32), r at tres; QKV tasks with
    // pub0 >= 0 also hand x's dimensions [pub0, pub0 + 64) on as tagged
    // words at tpub ([tiles*16][512]).
    const float *tmlp;
    int mlp_streams;
    uint64_t *tpub;
    int pub0;
    // EPI_GELU_W2 / EPI_SILU_W2: the MLP-out matrix (fragments, K = 2048 /
    // 512) and its scale plane (Q8); the task's partial goes to tmlp_out
    // ([mlp_streams][512] fp32, write-through).
    const void *w2;
    const uint16_t *w2scale;
    float *tmlp_out;
    // SRC_LN_MOD_PARTS: the previous block's gated residual, x = ln_x +
    // part_gate * ((P_0 + ... + P_7) + part_bias), P_j at tmlp + (j *
    // mlp_streams + s) * 512 and the gate row at part_gate + s *
    // ld_part_gate; dimensions [pub0, pub0 + 64) of x are stored at x_pub
    // ([streams][512]; null: none).
    const float *part_gate, *part_bias;
    int ld_part_gate;
    float *x_pub;
};

// ---------------------------------------------------------------------------
// Device-scope write-through stores (global_store sc1): visible in memory to
// every XCD once the wave's vmcnt drains.
__device__ inline void store_wt(float *p, float4 v) {
    const uint64_t lo = (uint64_t)fbits(v.x) | (uint64_t)fbits(v.y) << 32;
    const uint64_t hi = (uint64_t)fbits(v.z) | (uint64_t)fbits(v.w) << 32;
    __hip_atomic_store((uint64_t *)p, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store((uint64_t *)p + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline void store_wt(float2 *p, float2 v) {
    const uint64_t u = (uint64_t)fbits(v.x) | (uint64_t)fbits(v.y) << 32;
    __hip_atomic_store((uint64_t *)p, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline void store_wt(uint2 *p, uint2 v) {
    const uint64_t u = (uint64_t)v.x | (uint64_t)v.y << 32;
    __hip_atomic_store((uint64_t *)p, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A task output: write-through (read by tasks on other XCDs within the
// launch) or a plain store (read after the launch, or by tasks on the same
// XCD through its L2).
template <class T>
__device__ inline void store_out(T *p, T v, bool wt) {
    if (wt)
        store_wt(p, v);
    else
        *p = v;
}

__device__ inline void store_out(float *p, float4 v, bool wt) {
    if (wt)
        store_wt(p, v);
    else
        *(float4 *)p = v;
}

// 4 consecutive activations of stream s from column k (k % 4 == 0) as
// split fragments: three 8-byte stores.
// Only the first `terms` split terms are written (a consumer that reads two
// terms never reads the third).
// F16: the two fp16 terms of split2h in the first two records (terms is
// then ignored).
template <bool F16 = false>
__device__ inline void store_split4(uint16_t *__restrict__ xs, int s, int k, int kb_count,
                                    const float *v, bool wt, int terms = 3) {
    uint16_t h[4], m[4], l[4];
    if constexpr (F16) {
#pragma unroll
        for (int i = 0; i < 4; i++) split2h(v[i], h[i], m[i]);
        terms = 2;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) split3(v[i], h[i], m[i], l[i]);
    }
    const size_t base = split_index(s, k, 0, kb_count);
    store_out((uint2 *)(xs + base),
              make_uint2(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16), wt);
    store_out((uint2 *)(xs + base + 512),
              make_uint2(m[0] | (uint32_t)m[1] << 16, m[2] | (uint32_t)m[3] << 16), wt);
    if (terms == 3)
        store_out((uint2 *)(xs + base + 1024),
                  make_uint2(l[0] | (uint32_t)l[1] << 16, l[2] | (uint32_t)l[3] << 16), wt);
}

// ---------------------------------------------------------------------------
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
// LDS of a task: the prologue's operand buffer, reused for partial sums.
constexpr int kTaskLds = 16 * kLdsBlock;

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
    return xor16_32_sum(row16_sum(v));
}

// ---------------------------------------------------------------------------
// Prologues: 16 streams' 512-wide operand rows into LDS split fragments, by
// the task's 8 waves; wave w takes streams 2w and 2w+1 of the tile, lane j
// columns [8j, 8j+8) of each.

// Operand rows of the wave's two streams (2w, 2w+1 of tile st): lane j
// holds columns [8j, 8j+8); rows past `streams` read as zeros.
struct Rows2 {
    float v[2][8];
    bool live[2];
};

__device__ inline void rows_load(Rows2 &r, const float *x, int streams, int st) {
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int s = st * 16 + 2 * wave + i;
        r.live[i] = s < streams;  // uniform per wave
        if (r.live[i]) {
            const float4 x0 = *(const float4 *)(x + (size_t)s * kWidth + j * 8);
            const float4 x1 = *(const float4 *)(x + (size_t)s * kWidth + j * 8 + 4);
            r.v[i][0] = x0.x; r.v[i][1] = x0.y; r.v[i][2] = x0.z; r.v[i][3] = x0.w;
            r.v[i][4] = x1.x; r.v[i][5] = x1.y; r.v[i][6] = x1.z; r.v[i][7] = x1.w;
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) r.v[i][k] = 0.0f;
        }
    }
}

// rows_load from tagged rows (tile st's 16 rows of 512 words at `rows`):
// each wave polls its two streams' words until all carry the tag.
__device__ inline void rows_poll(Rows2 &r, const uint64_t *rows, int streams, int st,
                                 const TagPoll &tp) {
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rs = tag_rsrc(rows + (size_t)st * 16 * kWidth, 16 * kWidth * 8);
    u32x4 w[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++) r.live[i] = st * 16 + 2 * wave + i < streams;  // uniform
    const uint64_t t0 = wall_clock64();
    for (int round = 0;; round++) {
        __asm__ volatile("" ::: "memory");
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            if (!r.live[i]) continue;
            const uint32_t off = (uint32_t)(((2 * wave + i) * kWidth + 8 * j) * 8);
            const bool plain = round == 0 && tp.plain_first;
#pragma unroll
            for (int k = 0; k < 4; k++) w[i][k] = tag_load2(rs, off + 16 * k, plain);
#pragma unroll
            for (int k = 0; k < 4; k++) ok &= tag_ok2(w[i][k], tp.tag);
        }
        if (__all(ok)) break;
        if (tag_give_up(tp, t0, round)) break;
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            r.v[i][2 * k] = r.live[i] ? bitsf(w[i][k].x) : 0.0f;
            r.v[i][2 * k + 1] = r.live[i] ? bitsf(w[i][k].z) : 0.0f;
        }
}

// LayerNorm of the loaded rows, in place: two-pass fp32 moments per stream
// (one wave), then y = ((x - mean) * rstd) * w + b unfused, as the
// reference writes it (src/phonon_transformer.c:179-183); rows past the
// streams become zeros. Returns true if a live output is not finite.
__device__ inline bool rows_ln_values(Rows2 &r, const float *lw, const float *lb, float eps) {
    const int j = threadIdx.x & 63;
    const float4 w0 = *(const float4 *)(lw + j * 8), w1 = *(const float4 *)(lw + j * 8 + 4);
    const float4 b0 = *(const float4 *)(lb + j * 8), b1 = *(const float4 *)(lb + j * 8 + 4);
    const float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        float *u = r.v[i];
        const float mean =
            wave_sum64(((u[0] + u[1]) + (u[2] + u[3])) + ((u[4] + u[5]) + (u[6] + u[7]))) *
            (1.0f / kWidth);
        float q2[2] = {0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float c = __fsub_rn(u[k], mean);
            q2[k & 1] = fmaf(c, c, q2[k & 1]);
        }
        const float var = wave_sum64(q2[0] + q2[1]) * (1.0f / kWidth);
        const float rstd = 1.0f / sqrtf(var + eps);
        bool bad_i = false;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            u[k] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(u[k], mean), rstd), ws[k]), bs[k]);
            bad_i |= !isfinite(u[k]);
            if (!r.live[i]) u[k] = 0.0f;
        }
        bad |= bad_i && r.live[i];
    }
    return bad;
}

// rows_ln_values, then into the LDS operand buffer.
__device__ inline bool rows_ln(Rows2 &r, const float *lw, const float *lb, float eps,
                               uint16_t *bsh) {
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    const bool bad = rows_ln_values(r, lw, lb, eps);
#pragma unroll
    for (int i = 0; i < 2; i++) lds_store8(bsh, 2 * wave + i, j >> 2, j & 3, r.v[i]);
    return bad;
}

// The operands of rows_ln_mod_apply for the wave's two streams: the
// LayerNorm affine (lw, lb may be null) and the streams' shift and scale
// rows (shift at mod + s * ld, scale 512 further; rows past `streams` read
// the last stream's).
struct ModRows {
    float ws[8], bs[8];
    float4 m4[2][4];
    bool has_w, has_b;
};

__device__ inline void mod_load(ModRows &m, const float *lw, const float *lb, const float *mod,
                                int ld, int streams, int st) {
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    m.has_w = lw != nullptr;
    m.has_b = lb != nullptr;
    float4 w0 = make_float4(1.f, 1.f, 1.f, 1.f), w1 = w0;
    float4 b0 = make_float4(0.f, 0.f, 0.f, 0.f), b1 = b0;
    if (m.has_w) w0 = *(const float4 *)(lw + j * 8), w1 = *(const float4 *)(lw + j * 8 + 4);
    if (m.has_b) b0 = *(const float4 *)(lb + j * 8), b1 = *(const float4 *)(lb + j * 8 + 4);
    const float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int k = 0; k < 8; k++) m.ws[k] = ws[k], m.bs[k] = bs[k];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int s = min(st * 16 + 2 * wave + i, streams - 1);
        const float *sh = mod + (size_t)s * ld + j * 8;
        m.m4[i][0] = *(const float4 *)sh;
        m.m4[i][1] = *(const float4 *)(sh + 4);
        m.m4[i][2] = *(const float4 *)(sh + kWidth);
        m.m4[i][3] = *(const float4 *)(sh + kWidth + 4);
    }
}

// LayerNorm with the optional affine, then the adaLN modulation
// h * (1 + scale) + shift by the stream's own rows, in the element order of
// the flow head (src/phonon_sampler.c:250-278, 330-334, 350-354); fp32
// two-pass moments; into the LDS operand buffer. Returns true if a live
// output is not finite.
__device__ inline bool rows_ln_mod_apply(Rows2 &r, const ModRows &m, float eps, uint16_t *bsh) {
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        float *u = r.v[i];
        const float shift[8] = {m.m4[i][0].x, m.m4[i][0].y, m.m4[i][0].z, m.m4[i][0].w,
                                m.m4[i][1].x, m.m4[i][1].y, m.m4[i][1].z, m.m4[i][1].w};
        const float scale[8] = {m.m4[i][2].x, m.m4[i][2].y, m.m4[i][2].z, m.m4[i][2].w,
                                m.m4[i][3].x, m.m4[i][3].y, m.m4[i][3].z, m.m4[i][3].w};
        const float mean =
            wave_sum64(((u[0] + u[1]) + (u[2] + u[3])) + ((u[4] + u[5]) + (u[6] + u[7]))) *
            (1.0f / kWidth);
        float q2[2] = {0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float c = __fsub_rn(u[k], mean);
            q2[k & 1] = fmaf(c, c, q2[k & 1]);
        }
        const float var = wave_sum64(q2[0] + q2[1]) * (1.0f / kWidth);
        const float rstd = 1.0f / sqrtf(__fadd_rn(var, eps));
        bool bad_i = false;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            float h = __fmul_rn(__fsub_rn(u[k], mean), rstd);
            if (m.has_w) h = __fmul_rn(h, m.ws[k]);
            if (m.has_b) h = __fadd_rn(h, m.bs[k]);
            u[k] = __fadd_rn(__fmul_rn(h, __fadd_rn(1.0f, scale[k])), shift[k]);
            bad_i |= !isfinite(u[k]);
            if (!r.live[i]) u[k] = 0.0f;
        }
        bad |= bad_i && r.live[i];
        lds_store8(bsh, 2 * wave + i, j >> 2, j & 3, u);
    }
    return bad;
}

// mod_load, then rows_ln_mod_apply (every operand is requested before the
// first reduction).
__device__ inline bool rows_ln_mod(Rows2 &r, const float *lw, const float *lb, float eps,
                                   const float *mod, int ld, int streams, int st,
                                   uint16_t *bsh) {
    ModRows m;
    mod_load(m, lw, lb, mod, ld, streams, st);
    return rows_ln_mod_apply(r, m, eps, bsh);
}

// SRC_LN_MOD_PARTS (fused flow-head chain): the previous block's gated
// residual x = x_prev + gate * ((P_0 + P_1 + ... + P_7) + bias), its
// MLP-out dot given as the 8 partials of its MLP-in tasks (P_j covers hidden
// columns [64 j, 64 j + 64)). The partials are added in order, as
// gemm_split_task adds its 8 waves' column ranges at K = 512, and then the
// bias, gate and residual in EPI_GATED's order, so x has the bits of the
// unfused chain. Dimensions [pub0, pub0 + 64) of x go to x_pub (when set);
// then rows_ln_mod. Returns true if a live value is not finite.
__device__ inline bool prologue_ln_mod_parts(const GemmArgs &a, int st, uint16_t *bsh) {
    constexpr int P = kWidth / 64;
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    // Every operand is requested first: x_prev, the modulation rows, the
    // bias, then per stream its gate and partials (rows past the batch read
    // the last stream's; their results are never stored).
    Rows2 r;
    rows_load(r, a.ln_x, a.streams, st);
    ModRows m;
    mod_load(m, a.ln_w, a.ln_b, a.mod, a.ld_mod, a.streams, st);
    const bool has_b = a.part_bias != nullptr;
    float4 b0 = make_float4(0.f, 0.f, 0.f, 0.f), b1 = b0;
    if (has_b) {
        b0 = *(const float4 *)(a.part_bias + j * 8);
        b1 = *(const float4 *)(a.part_bias + j * 8 + 4);
    }
    const float bias[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const bool pub = a.x_pub && a.pub0 >= 0 && (j >> 3) == (a.pub0 >> 6);
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int s = min(st * 16 + 2 * wave + i, a.streams - 1);
        const float *g = a.part_gate + (size_t)s * a.ld_part_gate + j * 8;
        const float4 g0 = *(const float4 *)g, g1 = *(const float4 *)(g + 4);
        const float gate[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        float sum[8];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const float *q = a.tmlp + ((size_t)p * a.mlp_streams + s) * kWidth + j * 8;
            const float4 q0 = *(const float4 *)q, q1 = *(const float4 *)(q + 4);
            const float v[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
            for (int k = 0; k < 8; k++) sum[k] = p == 0 ? v[k] : __fadd_rn(sum[k], v[k]);
        }
        float *u = r.v[i];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float lin = has_b ? __fadd_rn(sum[k], bias[k]) : sum[k];
            u[k] = __fadd_rn(u[k], __fmul_rn(gate[k], lin));
            bad |= r.live[i] && !isfinite(u[k]);
        }
    }
    if (pub) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            if (!r.live[i]) continue;  // uniform per wave
            float *o = a.x_pub + (size_t)(st * 16 + 2 * wave + i) * kWidth + j * 8;
            const float *u = r.v[i];
            store_out(o, make_float4(u[0], u[1], u[2], u[3]), a.wt_out);
            store_out(o + 4, make_float4(u[4], u[5], u[6], u[7]), a.wt_out);
        }
    }
    bad |= rows_ln_mod_apply(r, m, a.ln_eps, bsh);
    return bad;
}

// The 16 streams' split fragments of tile st (K = 512) from global memory
// into the LDS operand buffer: 16 blocks of 1536 halves, each record in the
// same [term][lane][8] order.
__device__ inline void split_to_lds(const uint16_t *xs, int st, uint16_t *bsh) {
    const uint4 *src = (const uint4 *)(xs + (size_t)st * (kWidth / 32) * 1536);
    constexpr int per_block = 1536 / 8, total = (kWidth / 32) * per_block;
#pragma unroll
    for (int i0 = 0; i0 < total; i0 += kTaskThreads) {
        const int i = i0 + threadIdx.x;
        *(uint4 *)(bsh + (i / per_block) * kLdsBlock + (i % per_block) * 8) = src[i];
    }
}

// The loaded rows as they are (the merged attention output).
__device__ inline void rows_plain(const Rows2 &r, uint16_t *bsh) {
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 2; i++) lds_store8(bsh, 2 * wave + i, j >> 2, j & 3, r.v[i]);
}

// Merge of one (stream, head)'s split partials:
// out = sum_j acc_j e^(m_j - M) / sum_j l_j e^(m_j - M), M = max m_j (the
// normalisation after P.V of src/phonon_transformer.c:395-403), as a single
// pass in split order with a running maximum mx (the accumulators v are
// rescaled when it grows). merge_step folds in split j; the per-dimension
// arithmetic does not depend on how many dimensions a lane holds.
__device__ inline void merge_step(float &mx, float &total, float *v, int n, float m_j, float l_j,
                                  const float *acc_j) {
    const float m_new = fmaxf(mx, m_j);
    const float keep = expf(mx - m_new);  // 0 for the first split
    const float f = expf(m_j - m_new);
    mx = m_new;
    total = fmaf(l_j, f, total * keep);
    for (int i = 0; i < n; i++) v[i] = fmaf(acc_j[i], f, v[i] * keep);
}

// v /= total; returns true (and zeros) if the result is not finite or the
// sum is not positive.
template <int N>
__device__ inline bool merge_finish(float total, float *v) {
    bool bad = !(total > 0.0f) || !isfinite(total);
    const float inv = 1.0f / total;
#pragma unroll
    for (int i = 0; i < N; i++) {
        v[i] *= inv;
        bad |= !isfinite(v[i]);
    }
    if (bad) {
#pragma unroll
        for (int i = 0; i < N; i++) v[i] = 0.0f;
    }
    return bad;
}

// All splits of one (stream, head), dims [dim0, dim0 + N): split j's acc row
// is at acc + 64j, its (max, sum) at ml + 2j. Every load of a group of G
// splits is issued at once (one memory round trip per G splits); the result
// does not depend on G.
template <int N, int G = 8>
__device__ inline bool merge_splits(const float *acc, const float *ml, int nsplit, int dim0,
                                    float *v) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = 0.0f;
    float mx = -INFINITY, total = 0.0f;
    for (int j0 = 0; j0 < nsplit; j0 += G) {
        float2 ml8[G];
        float a8[G][N];
#pragma unroll
        for (int u = 0; u < G; u++) {
            const int js = min(j0 + u, nsplit - 1);
            ml8[u] = *(const float2 *)(ml + 2 * js);
#pragma unroll
            for (int k = 0; k < N / 4; k++) {
                const float4 q = *(const float4 *)(acc + js * 64 + dim0 + 4 * k);
                a8[u][4 * k] = q.x;
                a8[u][4 * k + 1] = q.y;
                a8[u][4 * k + 2] = q.z;
                a8[u][4 * k + 3] = q.w;
            }
        }
#pragma unroll
        for (int u = 0; u < G; u++) {
            if (j0 + u >= nsplit) break;
            merge_step(mx, total, v, N, ml8[u].x, ml8[u].y, a8[u]);
        }
    }
    return merge_finish<N>(total, v);
}

// Polls splits j0 .. nsplit-1 of one (stream, head) from its tagged partial
// records (lanes 0..15 of the wave: dims [4 lane, 4 lane + 4)) and folds
// them into the running merge in split order (merge_step: the arithmetic of
// merge_splits). Every lane of the wave must call it.
__device__ inline void merge_tagged_splits(const uint64_t *part, int j0, int nsplit, float &mx,
                                           float &total, float *v, const TagPoll &tp) {
    constexpr int G = 4;
    const int lane = threadIdx.x & 63;
    const bool mine = lane < 16;
    const __amdgpu_buffer_rsrc_t r =
        tag_rsrc(part, (uint32_t)(nsplit * PGPU_FLOW_PART_WORDS * 8));
    for (int g0 = j0; g0 < nsplit; g0 += G) {
        u32x4 acc[G][2], ml[G];
        const uint64_t t0 = wall_clock64();
        for (int round = 0;; round++) {
            __asm__ volatile("" ::: "memory");
            bool ok = true;
#pragma unroll
            for (int u = 0; u < G; u++) {
                const int j = min(g0 + u, nsplit - 1);
                const uint32_t rec = (uint32_t)(j * PGPU_FLOW_PART_WORDS * 8);
                if (mine) {
                    acc[u][0] = tag_load2(r, rec + lane * 32);
                    acc[u][1] = tag_load2(r, rec + lane * 32 + 16);
                    ml[u] = tag_load2(r, rec + 64 * 8);
                    ok &= tag_ok2(acc[u][0], tp.tag) && tag_ok2(acc[u][1], tp.tag) &&
                          tag_ok2(ml[u], tp.tag);
                }
            }
            if (__all(ok)) break;
            if (tag_give_up(tp, t0, round)) break;
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int u = 0; u < G; u++) {
            if (g0 + u >= nsplit) break;
            const float a4[4] = {bitsf(acc[u][0].x), bitsf(acc[u][0].z), bitsf(acc[u][1].x),
                                 bitsf(acc[u][1].z)};
            merge_step(mx, total, v, 4, bitsf(ml[u].x), bitsf(ml[u].z), a4);
        }
    }
}

// All splits of one (stream, head) from its tagged partial records, merged
// in split order with one dimension per lane (lane l: dimension l): the
// merge_step arithmetic, so dimension l gets the bits of merge_splits. Up
// to 8 records are requested per poll round (each lane its P.V word of
// each, lane u the record's max and sum, read back uniform), so a consumer
// that polls before the partials land sees them one round trip after the
// last one lands. Every lane of the wave must call it; returns true (and
// v = 0) if the result is not finite.
__device__ inline bool merge_tagged_dim(const uint64_t *part, int nsplit, const TagPoll &tp,
                                        float &v) {
    constexpr int G = 8;
    typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t r =
        tag_rsrc(part, (uint32_t)(nsplit * PGPU_FLOW_PART_WORDS * 8));
    float mx = -INFINITY, total = 0.0f;
    v = 0.0f;
    for (int g0 = 0; g0 < nsplit; g0 += G) {
        u32x2 acc[G];
        u32x4 ml;
        const uint32_t own = (uint32_t)(min(g0 + (lane & (G - 1)), nsplit - 1) *
                                        PGPU_FLOW_PART_WORDS * 8);
        const uint64_t t0 = wall_clock64();
        for (int round = 0;; round++) {
            __asm__ volatile("" ::: "memory");
            bool ok = true;
#pragma unroll
            for (int u = 0; u < G; u++) {
                const uint32_t rec = (uint32_t)(min(g0 + u, nsplit - 1) * PGPU_FLOW_PART_WORDS * 8);
                acc[u] = __builtin_amdgcn_raw_buffer_load_b64(r, rec + lane * 8, 0, 16);
                ok &= acc[u].y == tp.tag;
            }
            ml = tag_load2(r, own + 64 * 8);
            ok &= tag_ok2(ml, tp.tag);
            if (__all(ok)) break;
            if (tag_give_up(tp, t0, round)) break;
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int u = 0; u < G; u++) {
            if (g0 + u >= nsplit) break;
            const float m_j = bitsf(__builtin_amdgcn_readlane(ml.x, u));
            const float l_j = bitsf(__builtin_amdgcn_readlane(ml.z, u));
            const float a = bitsf(acc[u].x);
            merge_step(mx, total, &v, 1, m_j, l_j, &a);
        }
    }
    return merge_finish<1>(total, &v);
}

// The out projection's operand when it merges the attention splits itself
// (one-launch step, PGPU_FLOW_HANDOFF_MERGE_OUT): wave w merges head w of
// every live stream of tile st from the tagged partial records
// (merge_tagged_dim: lane l, dimension l) and writes the head's 64 values
// into the LDS operand buffer (column 64w + l: block 2w + l / 32, group
// (l % 32) / 8, element l % 8). A context the attention units cannot cover
// (they flag it and store nothing) and streams past the batch give zeros.
// `position`: lane n < 16 holds the position of stream n of the tile (loaded
// before the task's wait: positions are not written within the step).
__device__ inline bool prologue_attn_tagged(const GemmArgs &a, int st, int position,
                                            uint16_t *bsh) {
    const int h = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kb = 2 * h + (lane >> 5), g = (lane & 31) >> 3, e = lane & 7;
    bool bad = false;
#pragma unroll 1
    for (int n = 0; n < 16; n++) {
        const int s = st * 16 + n;
        float v = 0.0f;
        if (s < a.streams) {  // uniform
            const int count = __builtin_amdgcn_readlane(position, n) + 1;
            const int nsplit = (count + kSplitKeys - 1) / kSplitKeys;
            if (count >= 1 && nsplit <= a.max_splits && count <= a.table_stride * kBlockPos)
                bad |= merge_tagged_dim(
                    a.tparts + ((size_t)s * kHeads + h) * a.max_splits * PGPU_FLOW_PART_WORDS,
                    nsplit, a.tp, v);
        }
        uint16_t t[3];
        split3(v, t[0], t[1], t[2]);
        uint16_t *rec = bsh + kb * kLdsBlock + (g * 16 + n) * 8 + e;
#pragma unroll
        for (int p = 0; p < 3; p++) rec[p * 512] = t[p];
    }
    return bad;
}

// Merge of the split partials of 16 streams x 8 heads (layout of
// pgpu_attention_scratch): wave w merges streams 2w, 2w+1; lane
// (h = j/8, part = j%8) dims [8 part, 8 part + 8) of head h.
__device__ inline bool prologue_attn(const GemmArgs &a, int st, uint16_t *bsh) {
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    const int h = j >> 3, part = j & 7;
    bool bad = false;
#pragma unroll 1
    for (int i = 0; i < 2; i++) {
        const int n = 2 * wave + i, s = st * 16 + n;
        float v[8];
        if (s < a.streams) {
            const int count = a.positions[s] + a.pos_delta + 1;
            const int nsplit = min((count + kSplitKeys - 1) / kSplitKeys, a.max_splits);
            const size_t first = ((size_t)s * kHeads + h) * a.max_splits;
            bad |= merge_splits<8>(a.part_acc + first * 64, a.part_ml + first * 2, nsplit,
                                   part * 8, v);
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = 0.0f;
        }
        // Column 64h + 8 part: block 2h + part/4, group part%4.
        lds_store8(bsh, n, 2 * h + (part >> 2), part & 3, v);
    }
    return bad;
}

// Fused MLP (one-launch step, PGPU_FLOW_HANDOFF_FUSED_MLP): dimension d of
// stream s of a layer output, x = r + (P_0 + P_1 + ... + P_31). The MLP_IN
// tasks' partials (P_j at parts[(j * pstreams + s) * 512 + d]) are fp32
// values their tasks drained before counting: the caller has seen the count,
// so they are plain loads, shared through the XCD's L2 by the tasks that
// read them. r is the out projection's tagged row (r_row, the same in every
// lane of the wave), polled. Every lane of the wave must call it.
__device__ inline float fused_sum(const uint64_t *r_row, const float *parts, int pstreams, int s,
                                  int d, const TagPoll &tp) {
    constexpr int P = PGPU_FLOW_MLP_IN_TASKS;
    typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
    const __amdgpu_buffer_rsrc_t rr = tag_rsrc(r_row, (uint32_t)(kWidth * 8));
    const __amdgpu_buffer_rsrc_t rp =
        tag_rsrc(parts, (uint32_t)((size_t)P * pstreams * kWidth * sizeof(float)));
    // r's word and every partial in one round trip; r is polled again only
    // if its word does not carry the tag yet.
    u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rr, (uint32_t)(d * 8), 0, 16);
    const uint32_t off = (uint32_t)(((size_t)s * kWidth + d) * sizeof(float));
    const uint32_t step = (uint32_t)((size_t)pstreams * kWidth * sizeof(float));
    float v[P];
#pragma unroll
    for (int j = 0; j < P; j++)
        v[j] = bitsf(__builtin_amdgcn_raw_buffer_load_b32(rp, off, j * step, 0));
    const uint64_t t0 = wall_clock64();
    for (int round = 0; !__all(w.y == tp.tag); round++) {
        if (tag_give_up(tp, t0, round)) break;
        __builtin_amdgcn_s_sleep(1);
        __asm__ volatile("" ::: "memory");
        w = __builtin_amdgcn_raw_buffer_load_b64(rr, (uint32_t)(d * 8), 0, 16);
    }
    float sum = v[0];
#pragma unroll
    for (int j = 1; j < P; j++) sum = __fadd_rn(sum, v[j]);
    return __fadd_rn(bitsf(w.x), sum);  // residual + dot, as EPI_RESIDUAL
}

// SRC_LN_PARTS: the fused MLP's QKV prologue. For each live stream n of
// tile st (at most PGPU_FLOW_FUSED_MAX_STREAMS), thread d computes
// dimension d of the layer input x (fused_sum; dimensions [pub0, pub0 + 64)
// are handed on at tpub for the out projection's residual) and its
// LayerNorm (two-pass fp32 moments over the work-group, the waves' sums
// added in wave order; y = ((x - mean) * rstd) * w + b, as rows_ln_values)
// into an fp32 staging row; then each thread writes whole 16-byte split
// records of the LDS operand buffer (lds_store8: 8 columns of one stream),
// zeros for the streams past the batch. Returns true if a live output is
// not finite.
__device__ inline bool prologue_ln_parts(const GemmArgs &a, int st, uint16_t *bsh) {
    constexpr int N = PGPU_FLOW_FUSED_MAX_STREAMS;
    __shared__ float red[2][N][kTaskWaves];
    __shared__ __align__(16) float stage[N][kWidth];
    const int d = threadIdx.x, wave = d >> 6, lane = d & 63;
    const int live = min(N, a.streams - st * 16);
    const float lw = a.ln_w[d], lb = a.ln_b[d];
    const bool pub = a.tpub && a.pub0 >= 0 && d >= a.pub0 && d < a.pub0 + 64;
    float x[N];
#pragma unroll
    for (int n = 0; n < N; n++) {
        x[n] = 0.0f;
        if (n >= live) break;  // uniform
        const int s = st * 16 + n;
        x[n] = fused_sum(a.tres + (size_t)s * kWidth, a.tmlp, a.mlp_streams, s, d, a.tp);
        if (pub) store_tagged(a.tpub + (size_t)s * kWidth + d, x[n], a.tp.tag);
        const float sum = wave_sum64(x[n]);
        if (lane == 0) red[0][n][wave] = sum;
    }
    __syncthreads();
    float mean[N];
#pragma unroll
    for (int n = 0; n < N; n++) {
        mean[n] = 0.0f;
        if (n >= live) break;
        float t = red[0][n][0];
#pragma unroll
        for (int w = 1; w < kTaskWaves; w++) t = __fadd_rn(t, red[0][n][w]);
        mean[n] = t * (1.0f / kWidth);
        const float c = __fsub_rn(x[n], mean[n]);
        const float q = wave_sum64(__fmul_rn(c, c));
        if (lane == 0) red[1][n][wave] = q;
    }
    __syncthreads();
    bool bad = false;
#pragma unroll
    for (int n = 0; n < N; n++) {
        if (n >= live) break;
        float t = red[1][n][0];
#pragma unroll
        for (int w = 1; w < kTaskWaves; w++) t = __fadd_rn(t, red[1][n][w]);
        const float var = t * (1.0f / kWidth);
        const float rstd = 1.0f / sqrtf(var + a.ln_eps);
        const float y = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(x[n], mean[n]), rstd), lw), lb);
        bad |= !isfinite(y);
        stage[n][d] = y;
    }
    __syncthreads();
    // Records (stream n, 8-column group c): n = r % 16, c = r / 16.
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = threadIdx.x + i * kTaskThreads, n = r & 15, c = r >> 4;
        float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (n < live) {
            const float4 v0 = *(const float4 *)&stage[n][c * 8];
            const float4 v1 = *(const float4 *)&stage[n][c * 8 + 4];
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
        }
        lds_store8(bsh, n, c >> 2, c & 3, v);
    }
    return bad;
}

// ---------------------------------------------------------------------------
// Weights of one lane: CH column blocks.
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

// Blocks kb0 .. kb0+CH-1 of row tile `tile` of matrix (w, wscale) with kbn
// column blocks (clamped to kb_end - 1).
template <bool Q8, int CH>
__device__ inline void load_weights_of(WChunk<Q8, CH> &c, const void *w, const uint16_t *wscale,
                                       int tile, int kbn, int lane, int kb0, int kb_end) {
#pragma unroll
    for (int u = 0; u < CH; u++) {
        const size_t kb = (size_t)min(kb0 + u, kb_end - 1);
        if constexpr (Q8) {
            c.raw[u] = *(const uint2 *)((const int8_t *)w + ((size_t)tile * kbn + kb) * 512 +
                                        lane * 8);
            c.sc[u] = *(const uint2 *)(wscale + ((size_t)tile * kbn + kb) * 16 +
                                       (lane >> 4) * 4);
        } else {
            c.w[u] = *(const bf16x8 *)((const uint16_t *)w + ((size_t)tile * kbn + kb) * 512 +
                                       lane * 8);
        }
    }
}

// Makes the chunk's loads complete here: a task that is about to wait for
// its inputs then has its weights in registers for certain (the compiler
// may otherwise sink the loads past the wait, out of register pressure).
template <bool Q8, int CH>
__device__ inline void hold_weights(const WChunk<Q8, CH> &c) {
#pragma unroll
    for (int u = 0; u < CH; u++) {
        if constexpr (Q8)
            __asm__ volatile("" ::"v"(c.raw[u].x), "v"(c.raw[u].y), "v"(c.sc[u].x), "v"(c.sc[u].y));
        else
            __asm__ volatile("" ::"v"(c.w[u]));
    }
}

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

// acc += W_block . X_block for block u of a chunk; `used` false makes the
// block contribute 0 (scale 0 / zero fragment) with no control flow.
template <bool Q8, int CH>
__device__ inline void mfma_block(f32x4 &acc, const WChunk<Q8, CH> &w, int u, const bf16x8 &xh,
                                  const bf16x8 &xm, const bf16x8 &xl, bool used) {
    if constexpr (Q8) {
        const bf16x8 wa = q8_to_bf16(w.raw[u]);
        f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xh, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xm, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xl, c, 0, 0, 0);
        const uint2 s = used ? w.sc[u] : make_uint2(0u, 0u);
        acc[0] = fmaf(half_to_float(s.x & 0xffffu), c[0], acc[0]);
        acc[1] = fmaf(half_to_float(s.x >> 16), c[1], acc[1]);
        acc[2] = fmaf(half_to_float(s.y & 0xffffu), c[2], acc[2]);
        acc[3] = fmaf(half_to_float(s.y >> 16), c[3], acc[3]);
    } else {
        const bf16x8 wa = used ? w.w[u] : bf16x8{};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xm, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xl, acc, 0, 0, 0);
    }
}

// ---------------------------------------------------------------------------
// Epilogue operands of one lane (rows row0..row0+3 of stream s).
struct EpiOperands {
    float4 add;          // STORE, SILU_SPLIT, GATED: bias; RESIDUAL: residual
    bool has_add;
    float4 add2;         // SILU_SPLIT: bias2; GATED: residual
    bool has_add2;
    float4 gate;         // GATED
    float2 cs0, cs1;     // QKV: (cos, sin) of the lane's two RoPE pairs
    int pos, block;      // QKV: append position and its pool block
    bool ok;             // QKV: position and block are valid
};

// The K/V append slot of stream s: its position and pool block. Positions
// past the rope table or the block table, and block ids outside the pool,
// are errors: flagged by the epilogue, and nothing is written.
struct QkvSlot {
    int pos, block;
    bool ok;
};

__device__ inline QkvSlot qkv_slot(const GemmArgs &a, int s, bool live) {
    QkvSlot q{0, 0, false};
    if (!live) return q;
    int pos = a.positions[s] + a.pos_delta;
    q.ok = pos >= 0 && pos < kMaxPositions && (pos >> 4) < a.table_stride;
    if (q.ok) {
        q.block = a.tables[(size_t)s * a.table_stride + (pos >> 4)];
        q.ok = (unsigned)q.block < a.blocks;
    }
    q.pos = q.ok ? pos : 0;
    return q;
}

// The QKV epilogue's operands of rows row0..row0+3 at slot q: the slot and
// the RoPE phases of the lane's two interleaved pairs (those of position 0
// for a slot in error).
__device__ inline void qkv_operands(EpiOperands &e, const GemmArgs &a, const QkvSlot &q,
                                    int row0, bool live) {
    e.ok = live && q.ok;
    e.pos = q.pos;
    e.block = q.block;
    if (!live) return;
    const int d0 = (row0 & 511) & 63;
    e.cs0 = a.rope[(size_t)q.pos * 32 + (d0 >> 1)];
    e.cs1 = a.rope[(size_t)q.pos * 32 + (d0 >> 1) + 1];
}

// Operands that no task of the step writes (bias, positions, block tables,
// RoPE table): may be loaded before the task waits for its inputs.
template <int EPI>
__device__ inline void load_epilogue_static(EpiOperands &e, const GemmArgs &a, int s, int row0,
                                            bool live) {
    e.add = make_float4(0.f, 0.f, 0.f, 0.f);
    e.has_add = false;
    e.add2 = make_float4(0.f, 0.f, 0.f, 0.f);
    e.has_add2 = false;
    e.gate = make_float4(0.f, 0.f, 0.f, 0.f);
    e.ok = false;
    if (!live) return;
    if constexpr (EPI == EPI_STORE || EPI == EPI_SILU_SPLIT || EPI == EPI_GATED ||
                  EPI == EPI_SILU_W2) {
        if (a.bias) {
            e.add = *(const float4 *)(a.bias + row0);
            e.has_add = true;
        }
        if (EPI == EPI_SILU_SPLIT && a.bias2) {
            e.add2 = *(const float4 *)(a.bias2 + row0);
            e.has_add2 = true;
        }
    } else if constexpr (EPI == EPI_QKV) {
        qkv_operands(e, a, qkv_slot(a, s, true), row0, true);
    }
}

// Operands produced by earlier tasks of the step (the residual rows): loaded
// only after the task's wait (tagged residual rows: polled). Every lane of
// the wave must call it.
template <int EPI>
__device__ inline void load_epilogue_dynamic(EpiOperands &e, const GemmArgs &a, int st, int s,
                                             int row0, bool live) {
    if constexpr (EPI == EPI_RESIDUAL) {
        if (a.tres) {
            const __amdgpu_buffer_rsrc_t r =
                tag_rsrc(a.tres + (size_t)st * 16 * kWidth, 16 * kWidth * 8);
            e.add = poll_tagged4(r, (uint32_t)(((s & 15) * kWidth + row0) * 8), live, a.tp);
            e.has_add = live;
        } else if (live) {
            e.add = *(const float4 *)(a.residual + (size_t)s * a.ld_out + row0);
            e.has_add = true;
        }
    } else if constexpr (EPI == EPI_GATED) {
        if (a.tres) {  // tagged residual rows [tiles*16][512], polled
            const __amdgpu_buffer_rsrc_t r =
                tag_rsrc(a.tres + (size_t)st * 16 * kWidth, 16 * kWidth * 8);
            e.add2 = poll_tagged4(r, (uint32_t)(((s & 15) * kWidth + row0) * 8), live, a.tp);
            if (live) e.gate = *(const float4 *)(a.gate + (size_t)s * a.ld_gate + row0);
        } else if (live) {
            e.add2 = *(const float4 *)(a.residual + (size_t)s * a.ld_out + row0);
            e.gate = *(const float4 *)(a.gate + (size_t)s * a.ld_gate + row0);
        }
    }
}

// Consumer of one lane's four results v (rows row0..row0+3 of stream s).
// Returns true if a non-finite value was produced. FORMAT = kF16Pair (the
// fast prefill): the GELU outputs as fp16 pairs, with the fast GELU.
template <int EPI, int FORMAT = 3>
__device__ inline bool epilogue(const GemmArgs &a, const EpiOperands &e, const f32x4 &v, int s,
                                int row0, bool live) {
    bool bad = false;
    const bool wt = a.wt_out;
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
            if (a.tout)
                store_tagged4(a.tout + (size_t)s * kWidth + row0,
                              make_float4(y[0], y[1], y[2], y[3]), a.tp.tag);
            else
                store_out(o, make_float4(y[0], y[1], y[2], y[3]), wt);
        }
    } else if constexpr (EPI == EPI_GELU_SPLIT) {
        if (live) {
            float g[4];
            constexpr bool F16 = FORMAT == kF16Pair;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                g[r] = F16 ? gelu_erf_fast(v[r]) : gelu_erf(v[r]);
                bad |= !isfinite(g[r]);
            }
            store_split4<F16>(a.out_split, s, row0, a.out_kb, g, wt,
                              a.out_terms ? a.out_terms : 3);
        }
    } else if constexpr (EPI == EPI_SILU_SPLIT) {
        if (live) {
            const float add[4] = {e.add.x, e.add.y, e.add.z, e.add.w};
            const float add2[4] = {e.add2.x, e.add2.y, e.add2.z, e.add2.w};
            float g[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // bias + dot, then + bias2, then x / (1 + e^-x)
                float y = e.has_add ? __fadd_rn(v[r], add[r]) : v[r];
                if (e.has_add2) y = __fadd_rn(y, add2[r]);
                bad |= !isfinite(y);
                g[r] = __fdiv_rn(y, __fadd_rn(1.0f, expf(-y)));
                bad |= !isfinite(g[r]);
            }
            if (a.tout)  // fp32 tagged rows, split by the consumer
                store_tagged4(a.tout + (size_t)s * kWidth + row0,
                              make_float4(g[0], g[1], g[2], g[3]), a.tp.tag);
            else
                store_split4(a.out_split, s, row0, a.out_kb, g, wt);
        }
    } else if constexpr (EPI == EPI_GATED) {
        if (live) {
            float *o = a.out + (size_t)s * a.ld_out + row0;
            const float add[4] = {e.add.x, e.add.y, e.add.z, e.add.w};
            const float res[4] = {e.add2.x, e.add2.y, e.add2.z, e.add2.w};
            const float gate[4] = {e.gate.x, e.gate.y, e.gate.z, e.gate.w};
            float y[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float lin = e.has_add ? __fadd_rn(v[r], add[r]) : v[r];
                y[r] = __fadd_rn(res[r], __fmul_rn(gate[r], lin));
                bad |= !isfinite(y[r]);
            }
            if (a.tout)
                store_tagged4(a.tout + (size_t)s * kWidth + row0,
                              make_float4(y[0], y[1], y[2], y[3]), a.tp.tag);
            else
                store_out(o, make_float4(y[0], y[1], y[2], y[3]), wt);
            if (a.out_split) store_split4(a.out_split, s, row0, a.out_kb, y, wt);
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
            if (a.tqkv)  // every live lane, also for a flagged position
                store_tagged4(a.tqkv + (size_t)part * a.tqkv_part + (size_t)s * kWidth + rr,
                              part == 0 ? make_float4(o[0] * 0.125f, o[1] * 0.125f,
                                                      o[2] * 0.125f, o[3] * 0.125f)
                                        : make_float4(o[0], o[1], o[2], o[3]),
                              a.tp.tag);
            if (part == 0) {
                // The 1/sqrt(64) score scale is a power of two: folding it
                // into q is exact.
                store_out(a.q_out + (size_t)s * kWidth + rr,
                          make_float4(o[0] * 0.125f, o[1] * 0.125f, o[2] * 0.125f, o[3] * 0.125f),
                          !a.plain_qkv);
            } else if (ok) {
                float *dst = a.kv + (size_t)a.layer * a.layer_stride +
                             ((size_t)block * kHeads + head) * 2048 + (part - 1) * 1024 +
                             (pos & 15) * 64 + d0;
                store_out(dst, make_float4(o[0], o[1], o[2], o[3]), !a.plain_qkv);
            }
        }
    }
    return bad;
}

// The fused MLP's MLP-out weights of one wave (row tiles 4w .. 4w+3, the
// task's two column blocks of kbn); empty for every other epilogue.
template <bool Q8, bool ON>
struct W2Weights {
    WChunk<Q8, 2> w[4];
    __device__ void load(const GemmArgs &a, int bx, int wave, int lane, int kbn) {
#pragma unroll
        for (int u = 0; u < 4; u++)
            load_weights_of(w[u], a.w2, a.w2scale, wave * 4 + u, kbn, lane, 2 * bx, 2 * bx + 2);
    }
    __device__ void hold() const {
#pragma unroll
        for (int u = 0; u < 4; u++) hold_weights(w[u]);
    }
};
template <bool Q8>
struct W2Weights<Q8, false> {
    __device__ void load(const GemmArgs &, int, int, int, int) {}
    __device__ void hold() const {}
};

// EPI_GELU_W2 / EPI_SILU_W2 (fused MLP), after gemm_wide_task's half sums:
// the task's 64 activated rows (GELU of the dot; SiLU of dot + bias, as
// EPI_SILU_SPLIT) are hidden columns [64 bx, 64 bx + 64) of the MLP-out
// projection. Waves (t, half 0) put them into LDS as split fragments (two
// column blocks, past the half sums), then every wave multiplies its 4 row
// tiles of the MLP-out matrix by them (mfma_block: per-block Q8 order) and
// stores its rows of the task's partial write-through (the one-launch step
// drains them before it counts).
template <bool Q8, int EPI>
__device__ inline void act_w2_partial(const GemmArgs &a, uint16_t *bsh, const f32x4 &acc,
                                      const EpiOperands &e, const W2Weights<Q8, true> &w2, int t,
                                      int half, int s, bool live) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    uint16_t *hb = bsh + 2 * kLdsBlock;
    bool bad = false;
    if (half == 0) {
        const f32x4 p = ((const f32x4 *)bsh)[t * 64 + lane];
        const float add[4] = {e.add.x, e.add.y, e.add.z, e.add.w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float g;
            if constexpr (EPI == EPI_SILU_W2) {
                float y = __fadd_rn(acc[r], p[r]);
                if (e.has_add) y = __fadd_rn(y, add[r]);
                bad |= live && !isfinite(y);
                g = __fdiv_rn(y, __fadd_rn(1.0f, expf(-y)));
            } else {
                g = gelu_erf(__fadd_rn(acc[r], p[r]));
            }
            bad |= live && !isfinite(g);
            if (!live) g = 0.0f;
            const int c = 16 * t + (lane >> 4) * 4 + r;  // hidden column within the task
            uint16_t h, m, l;
            split3(g, h, m, l);
            uint16_t *rec = hb + (c >> 5) * kLdsBlock + ((c & 31) >> 3) * 128 + (lane & 15) * 8 +
                            (c & 7);
            rec[0] = h;
            rec[512] = m;
            rec[1024] = l;
        }
    }
    __syncthreads();
    bf16x8 xh[2], xm[2], xl[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint16_t *x = hb + u * kLdsBlock + lane * 8;
        xh[u] = *(const bf16x8 *)x;
        xm[u] = *(const bf16x8 *)(x + 512);
        xl[u] = *(const bf16x8 *)(x + 1024);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
        f32x4 y = {0.0f, 0.0f, 0.0f, 0.0f};
        mfma_block(y, w2.w[q], 0, xh[0], xm[0], xl[0], true);
        mfma_block(y, w2.w[q], 1, xh[1], xm[1], xl[1], true);
        if (live) {
            bad |= !isfinite(y[0]) || !isfinite(y[1]) || !isfinite(y[2]) || !isfinite(y[3]);
            store_wt(a.tmlp_out + (size_t)s * kWidth + (wave * 4 + q) * 16 + (lane >> 4) * 4,
                     make_float4(y[0], y[1], y[2], y[3]));
        }
    }
    flag_nonfinite(a.status, bad);
}

// A task's wait for its inputs: NoWait in the single-phase kernels. Every
// wait ends with a work-group barrier.
struct NoWait {
    __device__ void operator()() const { __syncthreads(); }
};

// ---------------------------------------------------------------------------
// Operand built by a prologue (K = 512): 4 row tiles (64 rows) x 16
// streams. The 8 waves each take (tile t = w%4, column half w/4): 8 blocks
// of 3 MFMAs, and the halves are added in order through LDS. The wave's
// weights and the epilogue's static operands are requested before the wait,
// so their latency overlaps it and the prologue (a projection task is on the
// step's latency-critical chain).
template <int SRC, int EPI, bool Q8, class Wait>
__device__ inline void gemm_wide_task(const GemmArgs &a, int bx, int st, uint16_t *bsh,
                                      const Wait &wait) {
    constexpr int kbn = kWidth / 32, KBW = kbn / 2;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t = wave & 3, half = wave >> 2;
    const int tile = bx * 4 + t;
    const bool active = tile < (a.n_rows >> 4);  // uniform per wave
    const int kb0 = half * KBW;
    const int s = st * 16 + (lane & 15);
    const bool live = s < a.streams;
    const int row0 = tile * 16 + (lane >> 4) * 4;

    WChunk<Q8, KBW> w;
    if (active) load_weights(w, a, tile, kbn, lane, kb0, kb0 + KBW);
    EpiOperands e;
    if (active && half == 0) load_epilogue_static<EPI>(e, a, s, row0, live);
    // The fused epilogue's MLP-out weights, requested with the projection's
    // own (the fused kernel runs one work-group per CU, so registers are
    // not what limits it).
    // The head's fused block (EPI_SILU_W2) requests them after its prologue
    // instead, whose loads they would otherwise queue behind.
    constexpr bool fused = EPI == EPI_GELU_W2 || EPI == EPI_SILU_W2;
    W2Weights<Q8, fused> w2;
    if constexpr (EPI == EPI_GELU_W2) w2.load(a, bx, wave, lane, kFfn / 32);
    if constexpr (SRC == SRC_LN_PARTS || EPI == EPI_GELU_W2)
        if (active) hold_weights(w);
    if constexpr (EPI == EPI_GELU_W2) w2.hold();
    int position = 0;
    if constexpr (SRC == SRC_ATTN_TAGGED)
        if (lane < 16 && st * 16 + lane < a.streams)
            position = a.positions[st * 16 + lane] + a.pos_delta;
    wait();
    if (active && half == 0) load_epilogue_dynamic<EPI>(e, a, st, s, row0, live);

    bool bad_in = false;
    if constexpr (SRC == SRC_ATTN) {
        bad_in = prologue_attn(a, st, bsh);
    } else if constexpr (SRC == SRC_ATTN_TAGGED) {
        bad_in = prologue_attn_tagged(a, st, position, bsh);
    } else if constexpr (SRC == SRC_SPLIT_LDS) {
        split_to_lds(a.xs, st, bsh);
    } else if constexpr (SRC == SRC_LN_PARTS) {
        bad_in = prologue_ln_parts(a, st, bsh);
    } else if constexpr (SRC == SRC_LN_MOD_PARTS) {
        bad_in = prologue_ln_mod_parts(a, st, bsh);
    } else {
        Rows2 r;
        if (a.tx)
            rows_poll(r, a.tx, a.streams, st, a.tp);
        else
            rows_load(r, a.ln_x, a.streams, st);
        if constexpr (SRC == SRC_LN)
            bad_in = rows_ln(r, a.ln_w, a.ln_b, a.ln_eps, bsh);
        else if constexpr (SRC == SRC_LN_MOD)
            bad_in = rows_ln_mod(r, a.ln_w, a.ln_b, a.ln_eps, a.mod, a.ld_mod, a.streams, st, bsh);
        else
            rows_plain(r, bsh);
    }
    flag_nonfinite(a.status, bad_in);
    if constexpr (EPI == EPI_SILU_W2) w2.load(a, bx, wave, lane, kWidth / 32);
    __syncthreads();
    if (a.ready_mark && threadIdx.x == 0) *a.ready_mark = wall_clock64();

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (active) {
#pragma unroll
        for (int c = 0; c < KBW / 4; c++) {
            bf16x8 xh[4], xm[4], xl[4];
            const uint16_t *xs = bsh + (kb0 + 4 * c) * kLdsBlock + lane * 8;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                xh[u] = *(const bf16x8 *)(xs + u * kLdsBlock);
                xm[u] = *(const bf16x8 *)(xs + u * kLdsBlock + 512);
                xl[u] = *(const bf16x8 *)(xs + u * kLdsBlock + 1024);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) mfma_block(acc, w, 4 * c + u, xh[u], xm[u], xl[u], true);
        }
    }
    // Half sums through LDS (the operand buffer is free once every wave has
    // its B operands).
    __syncthreads();
    f32x4 *partial = (f32x4 *)bsh;
    if (half == 1) partial[t * 64 + lane] = acc;
    __syncthreads();
    if constexpr (fused) {
        act_w2_partial<Q8, EPI>(a, bsh, acc, e, w2, t, half, s, live);
        return;
    }
    if (half == 0 && active) {
        const f32x4 p = partial[t * 64 + lane];
        f32x4 v;
        v[0] = __fadd_rn(acc[0], p[0]);
        v[1] = __fadd_rn(acc[1], p[1]);
        v[2] = __fadd_rn(acc[2], p[2]);
        v[3] = __fadd_rn(acc[3], p[3]);
        flag_nonfinite(a.status, epilogue<EPI>(a, e, v, s, row0, live));
    }
}

// Split-fragment rows from global memory (any K): one row tile x 16 streams.
// The 8 waves split the column blocks into 8 contiguous ranges (8 blocks
// each at K = 2048), in chunks of 4 with the next chunk's weights requested
// before the current chunk's MFMAs; the ranges are summed in LDS in wave
// order.
template <int EPI, bool Q8, class Wait>
__device__ inline void gemm_split_task(const GemmArgs &a, int tile, int st, uint16_t *lds,
                                       const Wait &wait) {
    constexpr int CH = 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int kbn = a.k_cols >> 5;
    const int per = (kbn + kTaskWaves - 1) / kTaskWaves;
    const int kb_begin = wave * per;
    const int kb_end = min(kbn, kb_begin + per);

    // D fragment of this lane: rows row0 .. row0+3 of stream s.
    const int s = st * 16 + (lane & 15);
    const int row0 = tile * 16 + (lane >> 4) * 4;
    const bool live = s < a.streams;

    WChunk<Q8, CH> w;
    if (kb_begin < kb_end) load_weights(w, a, tile, kbn, lane, kb_begin, kb_end);
    EpiOperands e;
    if (wave == 0) load_epilogue_static<EPI>(e, a, s, row0, live);
    wait();
    if (wave == 0) load_epilogue_dynamic<EPI>(e, a, st, s, row0, live);

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.tx && kb_begin < kb_end) {
        // Operand from tagged fp32 rows [tiles*16][512] (K = 512, at most 2
        // blocks per wave): lane (n, g) = (lane % 16, lane / 16) polls the 8
        // columns kb*32 + 8g .. +7 of stream st*16 + n for each of its
        // blocks and splits them as store_split4 would have (the same MFMA
        // operands, so the same bits as the fragment path).
        const __amdgpu_buffer_rsrc_t r =
            tag_rsrc(a.tx + (size_t)st * 16 * kWidth, 16 * kWidth * 8);
        u32x4 wv[2][4];
        const uint64_t t0 = wall_clock64();
        for (int round = 0;; round++) {
            __asm__ volatile("" ::: "memory");
            bool ok = true;
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const int kb = min(kb_begin + b, kb_end - 1);
                const uint32_t off =
                    (uint32_t)(((lane & 15) * kWidth + kb * 32 + 8 * (lane >> 4)) * 8);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (live) wv[b][q] = tag_load2(r, off + 16 * q, round == 0 && a.tp.plain_first);
                    ok &= !live || tag_ok2(wv[b][q], a.tp.tag);
                }
            }
            if (__all(ok)) break;
            if (tag_give_up(a.tp, t0, round)) break;
            __builtin_amdgcn_s_sleep(1);
        }
        bf16x8 xh[2], xm[2], xl[2];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            uint16_t h[8], m[8], l[8];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                split3(live ? bitsf(wv[b][q].x) : 0.0f, h[2 * q], m[2 * q], l[2 * q]);
                split3(live ? bitsf(wv[b][q].z) : 0.0f, h[2 * q + 1], m[2 * q + 1], l[2 * q + 1]);
            }
            xh[b] = __builtin_bit_cast(bf16x8, make_uint4(h[0] | (uint32_t)h[1] << 16,
                                                           h[2] | (uint32_t)h[3] << 16,
                                                           h[4] | (uint32_t)h[5] << 16,
                                                           h[6] | (uint32_t)h[7] << 16));
            xm[b] = __builtin_bit_cast(bf16x8, make_uint4(m[0] | (uint32_t)m[1] << 16,
                                                           m[2] | (uint32_t)m[3] << 16,
                                                           m[4] | (uint32_t)m[5] << 16,
                                                           m[6] | (uint32_t)m[7] << 16));
            xl[b] = __builtin_bit_cast(bf16x8, make_uint4(l[0] | (uint32_t)l[1] << 16,
                                                           l[2] | (uint32_t)l[3] << 16,
                                                           l[4] | (uint32_t)l[5] << 16,
                                                           l[6] | (uint32_t)l[7] << 16));
        }
        // The fragment path's chunk of CH blocks: blocks past the wave's
        // range repeat its last one with zero weights.
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const int b = min(u, 1);
            mfma_block(acc, w, u, xh[b], xm[b], xl[b], kb_begin + u < kb_end);
        }
    }
    const uint16_t *xs = a.xs + (size_t)st * kbn * 1536 + lane * 8;
    for (int kb0 = kb_begin; !a.tx && kb0 < kb_end; kb0 += CH) {
        // A lane whose stream is past the batch loads nothing: its MFMA
        // column is zero and its outputs are never stored.
        bf16x8 xh[CH], xm[CH], xl[CH];
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const size_t kb = (size_t)min(kb0 + u, kb_end - 1) * 1536;
            xh[u] = live ? *(const bf16x8 *)(xs + kb) : bf16x8{};
            xm[u] = live ? *(const bf16x8 *)(xs + kb + 512) : bf16x8{};
            xl[u] = live ? *(const bf16x8 *)(xs + kb + 1024) : bf16x8{};
        }
        WChunk<Q8, CH> next;
        if (kb0 + CH < kb_end) load_weights(next, a, tile, kbn, lane, kb0 + CH, kb_end);
#pragma unroll
        for (int u = 0; u < CH; u++) mfma_block(acc, w, u, xh[u], xm[u], xl[u], kb0 + u < kb_end);
        w = next;
    }

    f32x4 *partial = (f32x4 *)lds;
    partial[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave == 0) {
        f32x4 v = acc;
#pragma unroll
        for (int w2 = 1; w2 < kTaskWaves; w2++) {
            const f32x4 p = partial[w2 * 64 + lane];
            v[0] = __fadd_rn(v[0], p[0]);
            v[1] = __fadd_rn(v[1], p[1]);
            v[2] = __fadd_rn(v[2], p[2]);
            v[3] = __fadd_rn(v[3], p[3]);
        }
        flag_nonfinite(a.status, epilogue<EPI>(a, e, v, s, row0, live));
    }
}

}  // namespace pgpu
