// Batched causal prefill: every position of a prompt (or of several
// streams' prompts) through one layer at once, as large-M projections and a
// causal attention that reads each key block once per 64 queries
// (src/phonon_transformer.c:578-702, phonon_flow_stack_prefill, whose
// prefill_attention at :493-576 tiles queries against 512-key blocks).
//
// A layer is seven launches over the M pseudo-streams (one per position):
//   rows -> split   LayerNorm of the layer input into split fragments
//   QKV             projection, RoPE, q rows and the K/V append (pool)
//   attention       causal softmax(q K^T) V of every position, written as
//                   split fragments (or, exact mode, the decode step's split
//                   partials merged by the rows -> split pass)
//   OUT             projection + residual
//   rows -> split   LayerNorm of r
//   MLP_IN          projection + GELU, split fragments
//   MLP_OUT         projection + residual
//
// Projections. A work-group computes (8 R row tiles) x (P position tiles)
// of 16 x 16: wave w owns row tiles R w .. R w + R - 1 of the group and all
// P position tiles, whose split fragments (three bf16 terms per value) are
// staged in LDS one 32-column block at a time and read by all 8 waves. Each
// weight block is converted once and used for P position tiles. The
// arithmetic of every output is that of the decode step's tasks
// (pgpu_gemm.hpp): per 32-column block three MFMAs from zero and
// acc = fma(scale, c, acc) (Q8) or the MFMAs chained into acc (BF16), over
// chains of 8 blocks, and the chains summed in order (K = 512: the two
// halves of gemm_wide_task; K = 2048: the 8 wave ranges of gemm_split_task).
// So a prefill's projections give the bits of single steps.
//
// Attention (fast). One lane per query: a work-group of 4 waves takes 64
// consecutive positions of one stream and one head; wave w takes the key
// blocks b = w mod 4 of keys [0, last query], stages each block's K and V
// (16 keys x 64 x 2 fp32) in its LDS area, and keeps an online softmax
// (running max, sum and 64 accumulators) per lane in fp32. Keys past a
// lane's own position are skipped, never multiplied by a zero weight (pool
// slots past the context hold whatever they held). The four waves' states
// are merged in wave order through LDS, normalised and written as split
// fragments for the OUT projection. Its arithmetic differs from the decode
// step's in summation order only (fp32 throughout).
#include "pgpu_attention.hpp"
#include "pgpu_gemm.hpp"
#include "phonon_gpu.h"

namespace pgpu {
namespace {

// ---------------------------------------------------------------------------
// Rows -> split fragments: 16 rows per 512-thread work-group, through the
// decode step's own prologues (rows_ln: LayerNorm; prologue_attn: merge of
// the split-attention partials), then the LDS operand buffer is copied out
// in the global split layout (split_index, 16 column blocks).
template <int SRC>
__global__ __launch_bounds__(kTaskThreads) void k_rows_split(GemmArgs a, uint16_t *out) {
    __shared__ uint4 bsh4[kTaskLds / 8];
    uint16_t *bsh = (uint16_t *)bsh4;
    const int st = blockIdx.x;
    bool bad;
    if constexpr (SRC == SRC_ATTN) {
        bad = prologue_attn(a, st, bsh);
    } else {
        Rows2 r;
        rows_load(r, a.ln_x, a.streams, st);
        bad = rows_ln(r, a.ln_w, a.ln_b, a.ln_eps, bsh);
    }
    flag_nonfinite(a.status, bad);
    __syncthreads();
    constexpr int per_block = 1536 / 8, total = (kWidth / 32) * per_block;
    uint4 *dst = (uint4 *)(out + (size_t)st * (kWidth / 32) * 1536);
#pragma unroll
    for (int i0 = 0; i0 < total; i0 += kTaskThreads) {
        const int i = i0 + threadIdx.x;
        dst[i] = *(const uint4 *)(bsh + (i / per_block) * kLdsBlock + (i % per_block) * 8);
    }
}

// LayerNorm rows -> split fragments: one 16-row tile per 512-thread
// work-group. Wave w normalises rows 2w, 2w + 1 with the decode prologue's
// LayerNorm arithmetic (rows_ln_values: the same bits) into an LDS tile;
// then wave w writes column blocks 2w, 2w + 1: lane (g, n) = (lane / 16,
// lane % 16) splits row n, columns [8g, 8g + 8) of the block into its three
// terms, so that each term's 1 KB fragment record is one contiguous store.
// Only the first `terms` terms are written (the projections of a two-term
// prefill never read the third), or the two fp16 terms of kF16Pair. Rows
// past `streams` up to the tile's end become zeros.
constexpr int kLnTileStride = kWidth + 4;  // floats per LDS row: 8 lanes of a
                                           // 16-byte read hit distinct banks
__global__ __launch_bounds__(512) void k_rows_split_ln(const float *__restrict__ x,
                                                       const float *__restrict__ lw,
                                                       const float *__restrict__ lb, float eps,
                                                       int streams, int terms, uint16_t *out,
                                                       int *status) {
    __shared__ float4 tile4[16 * kLnTileStride / 4];
    float *tile = (float *)tile4;
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    const int st = blockIdx.x;
    Rows2 r;
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
    const bool bad = rows_ln_values(r, lw, lb, eps);
    flag_nonfinite(status, bad);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        float4 *row = (float4 *)(tile + (2 * wave + i) * kLnTileStride + j * 8);
        row[0] = make_float4(r.v[i][0], r.v[i][1], r.v[i][2], r.v[i][3]);
        row[1] = make_float4(r.v[i][4], r.v[i][5], r.v[i][6], r.v[i][7]);
    }
    __syncthreads();
    const int g = j >> 4, n = j & 15;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int kb = 2 * wave + i;
        const float4 *src = (const float4 *)(tile + n * kLnTileStride + kb * 32 + g * 8);
        const float4 v0 = src[0], v1 = src[1];
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        uint16_t h[8], m[8], l[8];
        if (terms == kF16Pair) {
#pragma unroll
            for (int k = 0; k < 8; k++) split2h(v[k], h[k], m[k]);
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) split3(v[k], h[k], m[k], l[k]);
        }
        uint16_t *rec = out + ((size_t)st * (kWidth / 32) + kb) * 1536 + j * 8;
#pragma unroll
        for (int p = 0; p < 3; p++) {
            if (p >= split_records(terms)) break;
            const uint16_t *t = p == 0 ? h : (p == 1 ? m : l);
            uint4 q;
            q.x = t[0] | (uint32_t)t[1] << 16;
            q.y = t[2] | (uint32_t)t[3] << 16;
            q.z = t[4] | (uint32_t)t[5] << 16;
            q.w = t[6] | (uint32_t)t[7] << 16;
            *(uint4 *)(rec + p * 512) = q;
        }
    }
}

// ---------------------------------------------------------------------------
// Large-M projection. A work-group computes RT = WR RW row tiles x PT = WP PW
// position tiles; wave (wr, wp) = (w / WP, w % WP) owns RW row tiles and PW
// position tiles of them. Every 32-column block's operands - the PT
// position tiles' split fragments (3 KB each), the RT row tiles' bf16 weight
// fragments (1 KB each) and, for Q8 weights, their fp32 row scales - are
// copied straight from global memory into one of NB LDS stages (LDS-DMA
// loads, 1 KB per wave instruction) NB - 1 blocks ahead of the MFMAs that
// use them, so the copies' latency overlaps NB - 1 blocks of MFMAs. The
// epilogue's operands (RoPE phases, block ids, residual rows; none is
// written by this launch) are loaded before the first block.
//
// Work-groups are dealt round-robin over the 8 XCDs, each with its own L2:
// when the position groups divide by 8, XCD x takes position groups
// x, x + 8, ... with all their row groups in turn, so the work-groups that
// share a position group's operand rows share an L2.
constexpr int kChain = 8;  // column blocks per summation chain

// One 16-byte LDS-DMA load per lane: global bytes [base + off, +16) -> LDS
// bytes [lds + 16 lane, +16) (base and lds wave-uniform, in SGPRs; off a
// per-lane byte offset). Issued as inline assembly so that the compiler,
// which cannot tell which LDS bytes such a load writes, does not drain
// every load in flight before each LDS read; the kernel's own vmcnt waits
// and barriers order the copies and the reads. M0 (the LDS base of the
// copy) is set right before the load; no other code of these kernels uses
// it (the compiler reserves M0 and does not take clobbers of it).
__device__ inline void dma16(const void *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(off), "s"(base), "s"(lds)
                 : "memory");
}

__device__ inline uint32_t lds_address(const void *p) {
    return __builtin_amdgcn_readfirstlane(
        (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)p);
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left alone).
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

// Waits until at most `later` blocks' loads of this wave are in flight,
// where the wave issues `per_block` loads per block (uniform; PER - 1, PER or
// PER + 1). Every count is an immediate: no per-stage scalar arithmetic.
template <int PER, int LATER>
__device__ inline void wait_blocks(int per_block) {
    if constexpr (LATER == 0) {
        wait_vm<0>();
    } else {
        if (per_block == PER) wait_vm<LATER * PER>();
        else if (per_block == PER + 1) wait_vm<LATER * (PER + 1)>();
        else if (per_block == PER - 1) wait_vm<LATER * (PER - 1)>();
        else wait_vm<0>();
    }
}

// TERMS: the split format (2 or 3 bf16 terms, or kF16Pair: two fp16 terms
// with fp16 weights on the fp16 matrix cores).
template <bool F16>
__device__ inline f32x4 mfma16(const bf16x8 &w, const bf16x8 &x, const f32x4 &c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, w),
                                                      __builtin_bit_cast(f16x8, x), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, x, c, 0, 0, 0);
}

template <int EPI, bool SCALED, int WR, int WP, int RW, int PW, int NB, int KS, int FORMAT>
__global__ __launch_bounds__(kTaskThreads) void k_prefill_gemm(GemmArgs a, int row_groups,
                                                               int pos_groups) {
    static_assert(FORMAT == 2 || FORMAT == 3 || FORMAT == kF16Pair, "split terms");
    constexpr int TERMS = split_records(FORMAT);
    constexpr bool F16 = FORMAT == kF16Pair;
    static_assert(WR * WP == kTaskWaves, "8 waves");
    static_assert(kChain % KS == 0, "a stage never straddles a chain");
    constexpr int RT = WR * RW, PT = WP * PW;
    constexpr int kB = PT * TERMS * 512, kA = RT * 512;     // halves per block
    constexpr int kS = SCALED ? RT * 32 : 0;                // halves (RT x 16 floats)
    constexpr int kBlk = kB + kA + kS;                      // halves per block
    constexpr int kStage = KS * kBlk;                       // halves per stage
    constexpr int kChunks = PT * TERMS + RT;                // 1 KB DMA chunks per block
    static_assert(!SCALED || RT * 4 <= 64, "one wave instruction moves the scales");
    __shared__ uint4 lds4[NB * kStage / 8];
    uint16_t *lds = (uint16_t *)lds4;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int wr = wave / WP, wp = wave % WP;
    const int kbn = a.k_cols >> 5;
    const int stages = kbn / KS;
    const int last_tile = (a.streams - 1) >> 4;
    int row_group, pos_group;
    if (pos_groups % 8 == 0) {
        const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
        pos_group = xcd + 8 * (local / row_groups);
        row_group = local % row_groups;
    } else {
        pos_group = blockIdx.x / row_groups;
        row_group = blockIdx.x % row_groups;
    }
    const int pt0 = pos_group * PT, rt0 = row_group * RT;
    const uint16_t *wv = (const uint16_t *)a.w;
    // This wave's share of every block's DMA chunks: chunk c = wave + 8 j.
    // Each keeps a running source pointer (uniform, advanced one block per
    // issue), its byte stride per block and its LDS offset within a block,
    // so that issuing a chunk is four scalar instructions and a load.
    constexpr int kPer = (kChunks + kTaskWaves - 1) / kTaskWaves;
    const char *csrc[kPer];
    uint32_t cstride[kPer], cdst[kPer];
    bool clive[kPer];
    int per_block = 0;  // loads this wave issues per block
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int c = wave + kTaskWaves * j;
        clive[j] = (kChunks % kTaskWaves == 0 || j < kPer - 1) ? true : c < kChunks;
        per_block += clive[j];
        if (c < PT * TERMS) {
            const int t = c / TERMS, term = c % TERMS;
            const int tile = min(pt0 + t, last_tile);
            csrc[j] = (const char *)(a.xs + (size_t)tile * kbn * 1536 + term * 512);
            cstride[j] = 1536 * 2;
            cdst[j] = (t * (TERMS * 512) + term * 512) * 2;
        } else {
            const int r = min(c - PT * TERMS, RT - 1);
            csrc[j] = (const char *)(wv + (size_t)(rt0 + r) * kbn * 512);
            cstride[j] = 512 * 2;
            cdst[j] = (kB + r * 512) * 2;
        }
    }
    // Q8 scales: wave 0, lane (r, part) -> the 16 bytes `part` of row tile
    // r's 16 row scales of the block.
    const char *ssrc = (const char *)(a.wscale_f + (size_t)rt0 * kbn * 16);
    const uint32_t soff = (uint32_t)((min(lane >> 2, RT - 1) * kbn * 16 + (lane & 3) * 4) * 4);
    if (SCALED && wave == 0) per_block++;
    const uint32_t lds0 = lds_address(lds);
    const uint32_t lane_off = lane * 16;
    int slot_next = 0;  // ring slot of the next stage issued

    auto issue = [&]() {
        const uint32_t sbase = lds0 + slot_next * (kStage * 2);
        slot_next = slot_next == NB - 1 ? 0 : slot_next + 1;
#pragma unroll
        for (int kk = 0; kk < KS; kk++) {
            const uint32_t bbase = sbase + kk * (kBlk * 2);
#pragma unroll
            for (int j = 0; j < kPer; j++) {
                if (clive[j]) dma16(csrc[j], lane_off, bbase + cdst[j]);
                csrc[j] += cstride[j];
            }
            if (SCALED && wave == 0) {
                if (lane < RT * 4) dma16(ssrc, soff, bbase + (kB + kA) * 2);
                ssrc += 64;
            }
        }
    };

    // acc: the running chain (reset at its end); tot: the chains
    // summed in order. tot starts at -0, the identity of fp32 addition, so
    // that adding the first chain gives that chain's bits exactly.
    f32x4 acc[RW][PW], tot[RW][PW];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int p = 0; p < PW; p++) {
            acc[r][p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            tot[r][p] = f32x4{-0.0f, -0.0f, -0.0f, -0.0f};
        }

    // Epilogue operands of every tile of the wave: requested first when the
    // wave holds at most 4 tiles; with more, after the main loop, where the
    // operand registers are free again.
    constexpr bool kLateEpi = RW * PW > 4;
    EpiOperands ep[RW][PW];
    auto load_epilogues = [&]() {
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int p = 0; p < PW; p++) {
                const int s = (pt0 + wp * PW + p) * 16 + (lane & 15);
                const int row0 = (rt0 + wr * RW + r) * 16 + (lane >> 4) * 4;
                load_epilogue_static<EPI>(ep[r][p], a, s, row0, s < a.streams);
                load_epilogue_dynamic<EPI>(ep[r][p], a, s >> 4, s, row0, s < a.streams);
            }
    };
    // Late QKV operands: a lane's append position and pool block depend on
    // its stream only (one per position tile), and are loaded before the
    // main loop; the RoPE phases they select follow it.
    QkvSlot qs[PW];
    if constexpr (kLateEpi && EPI == EPI_QKV) {
#pragma unroll
        for (int p = 0; p < PW; p++) {
            const int s = (pt0 + wp * PW + p) * 16 + (lane & 15);
            qs[p] = qkv_slot(a, s, s < a.streams);
        }
    }
    auto load_late_epilogues = [&]() {
        if constexpr (EPI == EPI_QKV) {
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int p = 0; p < PW; p++) {
                    const int s = (pt0 + wp * PW + p) * 16 + (lane & 15);
                    const int row0 = (rt0 + wr * RW + r) * 16 + (lane >> 4) * 4;
                    qkv_operands(ep[r][p], a, qs[p], row0, s < a.streams);
                }
        } else {
            load_epilogues();
        }
    };
    if constexpr (!kLateEpi) load_epilogues();

    // One 32-column block from LDS stage area st. Every tile's products
    // are issued term by term into its own registers (consecutive MFMAs
    // never depend on each other), then the Q8 scales are applied, one row
    // tile at a time (so that only PW tiles' block products are live).
    struct Frags {
        bf16x8 wa[RW], xt[PW][TERMS];
        float4 sc[RW];
    };
    auto load_frags = [&](Frags &f, const uint16_t *st) {
#pragma unroll
        for (int r = 0; r < RW; r++) {
            f.wa[r] = *(const bf16x8 *)(st + kB + (wr * RW + r) * 512 + lane * 8);
            if constexpr (SCALED)
                f.sc[r] = *(const float4 *)((const float *)(st + kB + kA) + (wr * RW + r) * 16 +
                                            (lane >> 4) * 4);
        }
#pragma unroll
        for (int p = 0; p < PW; p++)
#pragma unroll
            for (int t = 0; t < TERMS; t++)
                f.xt[p][t] =
                    *(const bf16x8 *)(st + (wp * PW + p) * (TERMS * 512) + t * 512 + lane * 8);
    };
    auto compute = [&](const Frags &f) {
        const auto &wa = f.wa;
        const auto &xt = f.xt;
        const auto &sc = f.sc;
        if constexpr (SCALED) {
#pragma unroll
            for (int r = 0; r < RW; r++) {
                f32x4 c[PW];
#pragma unroll
                for (int t = 0; t < TERMS; t++)
#pragma unroll
                    for (int p = 0; p < PW; p++)
                        c[p] = mfma16<F16>(wa[r], xt[p][t],
                                           t == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : c[p]);
#pragma unroll
                for (int p = 0; p < PW; p++) {
                    acc[r][p][0] = fmaf(sc[r].x, c[p][0], acc[r][p][0]);
                    acc[r][p][1] = fmaf(sc[r].y, c[p][1], acc[r][p][1]);
                    acc[r][p][2] = fmaf(sc[r].z, c[p][2], acc[r][p][2]);
                    acc[r][p][3] = fmaf(sc[r].w, c[p][3], acc[r][p][3]);
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < TERMS; t++)
#pragma unroll
                for (int r = 0; r < RW; r++)
#pragma unroll
                    for (int p = 0; p < PW; p++)
                        acc[r][p] = mfma16<F16>(wa[r], xt[p][t], acc[r][p]);
        }
    };
    auto block = [&](const uint16_t *st) {
        Frags f;
        load_frags(f, st);
        compute(f);
        // The next block's code is not scheduled into this one: that would
        // keep two blocks' products and operands live at once.
        __builtin_amdgcn_sched_barrier(0);
    };
    auto chain_end = [&](int blocks_done) {
        if ((blocks_done & (kChain - 1)) == 0) {
            // End of a chain: the chains are summed in order.
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int p = 0; p < PW; p++) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        tot[r][p][e] = __fadd_rn(tot[r][p][e], acc[r][p][e]);
                    acc[r][p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                }
        }
    };

    for (int k = 0; k < NB - 1 && k < stages; k++) issue();
    int slot = 0;  // ring slot of stage sg
    for (int sg = 0; sg < stages; sg++) {
        // Stage sg is in once at most the later stages' loads are in
        // flight (all of them issued while sg + NB - 2 < stages; in the
        // last stages every load is waited for); the barrier publishes
        // every wave's copies and frees the stage the next issue
        // overwrites (read in the previous iteration).
        if (sg + NB - 2 < stages) wait_blocks<kPer, (NB - 2) * KS>(per_block);
        else wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        if (sg + NB - 1 < stages) issue();
        const uint16_t *st = lds + slot * kStage;
        slot = slot == NB - 1 ? 0 : slot + 1;
#pragma unroll
        for (int kk = 0; kk < KS; kk++) block(st + kk * kBlk);
        chain_end((sg + 1) * KS);
    }

    if constexpr (kLateEpi) load_late_epilogues();
    bool bad = false;
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int p = 0; p < PW; p++) {
            const int s = (pt0 + wp * PW + p) * 16 + (lane & 15);
            const int row0 = (rt0 + wr * RW + r) * 16 + (lane >> 4) * 4;
            bad |= epilogue<EPI, FORMAT>(a, ep[r][p], tot[r][p], s, row0, s < a.streams);
        }
    flag_nonfinite(a.status, bad);
}

// Q8 fragments to bf16 fragments (the same order; int8 values are exact in
// bf16), optionally to fp16 fragments too, and fp16 block scales to fp32
// (exact).
__global__ void k_wide_from_q8(const int8_t *__restrict__ values, const uint16_t *__restrict__ scales,
                               size_t n_values, uint16_t *__restrict__ out_values,
                               float *__restrict__ out_scales, uint16_t *__restrict__ out_f16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_values / 8; i += stride) {
        const uint2 raw = *(const uint2 *)(values + i * 8);
        *(bf16x8 *)(out_values + i * 8) = q8_to_bf16(raw);
        if (out_f16) {
            // int8 values are exact in fp16 as well
            f16x8 h;
#pragma unroll
            for (int k = 0; k < 8; k++)
                h[k] = (_Float16)(float)(int8_t)((k < 4 ? raw.x : raw.y) >> (8 * (k & 3)));
            *(f16x8 *)(out_f16 + i * 8) = h;
        }
    }
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_values / 32; i += stride)
        out_scales[i] = half_to_float(scales[i]);
}

// ---------------------------------------------------------------------------
// Fast causal attention. entries: [count][2] (s0, n): pseudo-streams
// s0 .. s0 + n - 1 (n <= 64) are consecutive positions of one stream and
// share the block table row of s0. Grid (entries, heads), 4 waves.
constexpr int kAttnWaves = 4;
constexpr int kQueries = PGPU_PREFILL_RUN;
static_assert(kQueries == 64, "one lane per query of a run");
// LDS per wave: one key block's K then V (16 x 64 fp32 each); after the
// key loop the same array holds waves 1..3's (max, sum, 64 accumulators).
constexpr int kWaveKv = 2 * kBlockPos * kHeadDim;
constexpr int kMergeFloats = (kAttnWaves - 1) * (2 + kHeadDim) * 64;
constexpr int kAttnLds = kMergeFloats > kAttnWaves * kWaveKv ? kMergeFloats : kAttnWaves * kWaveKv;

__global__ __launch_bounds__(64 * kAttnWaves) void k_prefill_attention_rows(
    const float *__restrict__ q, const float *__restrict__ kv, size_t layer_stride,
    unsigned blocks, int layer, const int32_t *__restrict__ tables, int table_stride,
    const int32_t *__restrict__ positions, int streams, const int32_t *__restrict__ entries,
    uint16_t *__restrict__ out_split, int terms, int *status) {
    __shared__ float4 lds4[kAttnLds / 4];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int head = blockIdx.y;
    const int s0 = entries[2 * blockIdx.x], n = entries[2 * blockIdx.x + 1];
    // A malformed entry is flagged and computes nothing.
    if (n < 1 || n > kQueries || s0 < 0 || s0 > streams - n) {
        if (threadIdx.x == 0) atomicOr(status, 2);
        return;
    }
    const int p0 = positions[s0];
    const int p_last = p0 + n - 1;
    const bool mine = lane < n;
    const int pos = p0 + lane;
    const int32_t *table = tables + (size_t)s0 * table_stride;
    const float *layer_kv = kv + (size_t)layer * layer_stride;

    float qv[kHeadDim];
    {
        const float *qrow = q + (size_t)(s0 + (mine ? lane : 0)) * kWidth + head * kHeadDim;
#pragma unroll
        for (int d = 0; d < kHeadDim; d += 4) {
            const float4 v = *(const float4 *)(qrow + d);
            qv[d] = v.x;
            qv[d + 1] = v.y;
            qv[d + 2] = v.z;
            qv[d + 3] = v.w;
        }
    }
    float acc[kHeadDim];
#pragma unroll
    for (int d = 0; d < kHeadDim; d++) acc[d] = 0.0f;
    float m = -INFINITY, l = 0.0f;

    float4 *mine_kv = lds4 + wave * (kWaveKv / 4);
    // A context the block table cannot cover is an error: flagged, and only
    // the covered keys are read.
    if (p_last / kBlockPos >= table_stride && wave == 0 && lane == 0) atomicOr(status, 2);
    const int nblocks = min(p_last / kBlockPos + 1, table_stride);
    bool bad_block = false;
    // Keys of block b: the wave's 64 lanes move its K then V tile (1024
    // floats each, contiguous in the pool) with four 16-byte loads per lane.
    float4 n0, n1, n2, n3, n4, n5, n6, n7;
#define PGPU_FETCH_KV(b_)                                                                    \
    do {                                                                                     \
        int id_ = table[(b_)];                                                               \
        bad_block |= (unsigned)id_ >= blocks;                                                \
        id_ = (unsigned)id_ < blocks ? id_ : 0;                                              \
        const float4 *t_ = (const float4 *)(layer_kv + ((size_t)id_ * kHeads + head) * 2048) + \
                           lane;                                                             \
        n0 = t_[0];                                                                          \
        n1 = t_[64];                                                                         \
        n2 = t_[128];                                                                        \
        n3 = t_[192];                                                                        \
        n4 = t_[256];                                                                        \
        n5 = t_[320];                                                                        \
        n6 = t_[384];                                                                        \
        n7 = t_[448];                                                                        \
    } while (0)
    int b = wave;
    if (b < nblocks) PGPU_FETCH_KV(b);
    for (; b < nblocks; b += kAttnWaves) {
        mine_kv[lane] = n0;
        mine_kv[64 + lane] = n1;
        mine_kv[128 + lane] = n2;
        mine_kv[192 + lane] = n3;
        mine_kv[256 + lane] = n4;
        mine_kv[320 + lane] = n5;
        mine_kv[384 + lane] = n6;
        mine_kv[448 + lane] = n7;
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
        __builtin_amdgcn_wave_barrier();
        if (b + kAttnWaves < nblocks) PGPU_FETCH_KV(b + kAttnWaves);
        const float *kt = (const float *)mine_kv;
        const float *vt = kt + kBlockPos * kHeadDim;
        const int key0 = b * kBlockPos;
        const bool full = key0 + kBlockPos - 1 <= p0;  // every key at or before every query
        float sc[kBlockPos];
        float bm = -INFINITY;
#pragma unroll
        for (int j = 0; j < kBlockPos; j++) {
            float dot = 0.0f;
#pragma unroll
            for (int d = 0; d < kHeadDim; d += 4) {
                const float4 k = *(const float4 *)(kt + j * kHeadDim + d);
                dot = fmaf(qv[d], k.x, dot);
                dot = fmaf(qv[d + 1], k.y, dot);
                dot = fmaf(qv[d + 2], k.z, dot);
                dot = fmaf(qv[d + 3], k.w, dot);
            }
            const bool use = full || key0 + j <= pos;
            sc[j] = use ? dot : -INFINITY;
            bm = fmaxf(bm, sc[j]);
        }
        if (mine && bm > -INFINITY) {
            const float mn = fmaxf(m, bm);
            const float keep = expf(m - mn);  // 0 on the first block
            m = mn;
            l *= keep;
#pragma unroll
            for (int d = 0; d < kHeadDim; d++) acc[d] *= keep;
#pragma unroll
            for (int j = 0; j < kBlockPos; j++) {
                if (sc[j] == -INFINITY) continue;
                const float e = expf(sc[j] - mn);
                l += e;
#pragma unroll
                for (int d = 0; d < kHeadDim; d += 4) {
                    const float4 v = *(const float4 *)(vt + j * kHeadDim + d);
                    acc[d] = fmaf(e, v.x, acc[d]);
                    acc[d + 1] = fmaf(e, v.y, acc[d + 1]);
                    acc[d + 2] = fmaf(e, v.z, acc[d + 2]);
                    acc[d + 3] = fmaf(e, v.w, acc[d + 3]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // every lane is done with the tile
    }
#undef PGPU_FETCH_KV
    if (bad_block) atomicOr(status, 2);

    // Merge the four waves' states in wave order: waves 1..3 publish
    // (m, l, acc) per lane, wave 0 folds them in.
    __syncthreads();
    float *pub = (float *)lds4;  // [wave-1][66][64]
    if (wave > 0) {
        float *dst = pub + (size_t)(wave - 1) * 66 * 64;
        dst[lane] = m;
        dst[64 + lane] = l;
#pragma unroll
        for (int d = 0; d < kHeadDim; d++) dst[(2 + d) * 64 + lane] = acc[d];
    }
    __syncthreads();
    if (wave != 0 || !mine) return;
#pragma unroll 1
    for (int w = 1; w < kAttnWaves; w++) {
        const float *src = pub + (size_t)(w - 1) * 66 * 64;
        const float mw = src[lane];
        if (mw == -INFINITY) continue;  // the wave saw no key of this lane
        const float lw = src[64 + lane];
        const float mn = fmaxf(m, mw);
        const float keep = expf(m - mn), f = expf(mw - mn);
        m = mn;
        l = fmaf(lw, f, l * keep);
#pragma unroll
        for (int d = 0; d < kHeadDim; d++) acc[d] = fmaf(src[(2 + d) * 64 + lane], f, acc[d] * keep);
    }
    const bool ok = l > 0.0f && isfinite(l);
    const float inv = 1.0f / l;
    bool bad = !ok;
#pragma unroll
    for (int d = 0; d < kHeadDim; d += 4) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = ok ? acc[d + i] * inv : 0.0f;
            bad |= !isfinite(v[i]);
        }
        if (terms == kF16Pair)
            store_split4<true>(out_split, s0 + lane, head * kHeadDim + d, kWidth / 32, v, false);
        else
            store_split4(out_split, s0 + lane, head * kHeadDim + d, kWidth / 32, v, false, terms);
    }
    flag_nonfinite(status, bad);
}

// ---------------------------------------------------------------------------
// Causal attention of a pair of runs (each up to 64 consecutive positions)
// of one stream and one head on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32): waves 0-3 take the first run, waves 4-7 the
// second (none if its count is 0), wave 16w .. 16w+15 of its run's queries.
// The host pairs a stream's run with the most keys with the one with the
// fewest, so that every work-group does about the same work under the
// causal mask. The pair's keys go through LDS in chunks of 64 (four pool
// blocks, K and V), each chunk loaded once by the work-group and consumed
// by every wave that needs it: per 16-key sub-block a wave computes
// S^T = K Q^T (16 MFMAs over the 64 dimensions; lane l holds keys
// 4(l/16) .. +3 of query l%16); then, once per chunk, an online softmax step
// per query (the query's scores sit in the 4 lanes l%16 + 16g) and O^T +=
// V^T P^T (16 MFMAs per sub-block: the P^T operand is the S^T registers
// themselves). Products are exact fp32 multiplications; sums are in the
// matrix cores' order. A query's arithmetic does not depend on the run it
// is paired with.
//
// FAST (the fast prefill): the products on the 16-bit matrix cores.
// - S^T = K Q^T with q and K each split into three bf16 terms (split3: 24
//   significant bits, fp32's exponent range) and the six products
//   m.m + l.h + h.l + m.h + h.m + h.h (the dropped ones are 2^-24 of the
//   product): 12 v_mfma_f32_16x16x32_bf16 per 16-key sub-block. The scores
//   are the sensitive part (at the benchmark weights they reach tens, and
//   their error moves every probability): two fp16 terms (22 bits) there
//   put 4x the fp32 kernel's distance from the oracle at the end of the
//   12-layer stack.
// - O^T += V^T P^T with V and P each split into two fp16 terms, hi =
//   fp16(x), lo = fp16(x - hi) (22 significant bits, 5e-7 of the output),
//   and the products hi.hi + hi.lo + lo.hi: 3 v_mfma_f32_16x16x32_f16 per
//   (16-dimension tile, 32 keys). P is scaled by 2^12 before its split
//   (exact; P <= 1) so that the lo terms of small probabilities stay out of
//   fp16's subnormal range; the output's normalisation takes the 2^-12 back.
//   A value of magnitude 65520 or more overflows fp16 and makes the output
//   non-finite, which the status word reports.
// K goes into LDS as [key][h 64 | m 64 | l 64] and V transposed,
// [dimension][hi 64 keys | lo 64 keys], so that every operand is one or two
// LDS reads. The 32 keys of a value step are the lane's keys 4g .. 4g+3 of
// two sub-blocks (the slots of the score registers): V^T's lanes read the
// same keys.
constexpr int kMmaKeys = 64;                 // keys per LDS chunk
constexpr int kMmaRow = kHeadDim + 4;        // padded LDS row (floats)
constexpr int kF16Row = 2 * kMmaRow;         // FAST V^T row (halves): hi 64 | lo 64 | pad
constexpr int kKRow = 3 * kHeadDim + 8;      // FAST K row (bf16): h 64 | m 64 | l 64 | pad
constexpr int kPairThreads = 512;
constexpr float kPScale = 4096.0f;           // FAST: P is split as P * 2^12

__device__ inline f16x8 f16x8_of(uint2 a, uint2 b) {
    return __builtin_bit_cast(f16x8, make_uint4(a.x, a.y, b.x, b.y));
}

template <bool FAST>
__global__ __launch_bounds__(kPairThreads) void k_prefill_attention_mfma(
    const float *__restrict__ q, const float *__restrict__ kv, size_t layer_stride,
    unsigned blocks, int layer, const int32_t *__restrict__ tables, int table_stride,
    const int32_t *__restrict__ positions, int streams, const int32_t *__restrict__ pairs,
    uint16_t *__restrict__ out_split, int terms, int *status) {
    __shared__ __align__(16) float kt[FAST ? kMmaKeys * kKRow / 2 : kMmaKeys * kMmaRow];
    __shared__ __align__(16) float vt[kMmaKeys * kMmaRow];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, t = threadIdx.x;
    const int head = blockIdx.y, half = wave >> 2, hw = wave & 3;
    const int s0a = pairs[4 * blockIdx.x], na = pairs[4 * blockIdx.x + 1];
    const int s0b = pairs[4 * blockIdx.x + 2], nb = pairs[4 * blockIdx.x + 3];
    if (na < 1 || na > kQueries || s0a < 0 || s0a > streams - na || nb < 0 || nb > kQueries ||
        (nb > 0 && (s0b < 0 || s0b > streams - nb))) {
        if (t == 0) atomicOr(status, 2);
        return;  // uniform over the work-group
    }
    // Both runs are positions of one stream: they share its block table.
    const int32_t *table = tables + (size_t)s0a * table_stride;
    const float *layer_kv = kv + (size_t)layer * layer_stride;
    // Block-table entries go one chunk ahead of the K/V loads, and the first
    // chunks' entries and K/V are requested before the runs' positions are
    // known (every index stays inside the table and the pool; keys past the
    // pair's last position are zeroed when the chunk is stored in LDS).
    constexpr int kChunkBlocks = kMmaKeys / kBlockPos;
    int ids[kChunkBlocks], next_ids[kChunkBlocks];
#pragma unroll
    for (int b = 0; b < kChunkBlocks; b++) {
        ids[b] = b < table_stride ? table[b] : 0;
        next_ids[b] = kChunkBlocks + b < table_stride ? table[kChunkBlocks + b] : 0;
    }
    // Thread t moves float4 t of each of the chunk's pool blocks' (K | V)
    // pair (K: float4 0 .. 255, V: 256 .. 511). FAST: the V threads take
    // the float4s column-wise instead (position t % 16, dimensions
    // 4 ((t - 256) / 16) .. +3), so that the lanes of a wave write
    // consecutive keys of one dimension into the transposed V.
    const int fidx = FAST && t >= 256 ? 256 + ((t & 15) << 4) + ((t - 256) >> 4) : t;
    float4 pre[kChunkBlocks];
#define PGPU_FETCH_CHUNK()                                                                  \
    do {                                                                                    \
        _Pragma("unroll") for (int i = 0; i < kChunkBlocks; i++) {                          \
            const int id_ = ids[i];                                                         \
            const int safe_ = (unsigned)id_ < blocks ? id_ : 0;                             \
            const float *blk_ = layer_kv + ((size_t)safe_ * kHeads + head) * 2048;          \
            pre[i] = ((const float4 *)blk_)[fidx];                                          \
        }                                                                                   \
    } while (0)
    PGPU_FETCH_CHUNK();
    const int pa = positions[s0a], pb = nb > 0 ? positions[s0b] : 0;
    const int p_last = max(pa + na - 1, nb > 0 ? pb + nb - 1 : -1);
    if (p_last / kBlockPos >= table_stride && t == 0) atomicOr(status, 2);
    const int key_end = min(p_last + 1, table_stride * kBlockPos);  // keys [0, key_end)
    const int chunks = (key_end + kMmaKeys - 1) / kMmaKeys;
    bool bad_block = false;
    // This wave's run.
    const int s0 = half ? s0b : s0a, n = half ? nb : na, p0 = half ? pb : pa;

    // This lane's query (column l%16 of the wave's 16) and its 16 dimensions
    // 16(l/16) .. +15: the B operand of S^T = K Q^T, one dimension per MFMA.
    const int qi = hw * 16 + (lane & 15), g = lane >> 4;
    const bool q_live = qi < n;
    const int qpos = p0 + qi;
    float qv[16];
    // FAST: the lane's dimensions 32h + 8g .. +7 (h = 0, 1) as three bf16
    // terms q3[term][h].
    bf16x8 q3[3][2];
    if constexpr (FAST) {
        const float *src =
            q + (size_t)(s0 + (q_live ? qi : 0)) * kWidth + head * kHeadDim + 8 * g;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 a = *(const float4 *)(src + 32 * h);
            const float4 b = *(const float4 *)(src + 32 * h + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            uint16_t t3[3][8];
#pragma unroll
            for (int j = 0; j < 8; j++) split3(q_live ? v[j] : 0.0f, t3[0][j], t3[1][j], t3[2][j]);
#pragma unroll
            for (int p = 0; p < 3; p++)
                q3[p][h] = __builtin_bit_cast(
                    bf16x8, make_uint4(t3[p][0] | (uint32_t)t3[p][1] << 16,
                                       t3[p][2] | (uint32_t)t3[p][3] << 16,
                                       t3[p][4] | (uint32_t)t3[p][5] << 16,
                                       t3[p][6] | (uint32_t)t3[p][7] << 16));
        }
    } else {
        const float4 *src = (const float4 *)(q + (size_t)(s0 + (q_live ? qi : 0)) * kWidth +
                                             head * kHeadDim + 16 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = src[i];
            qv[4 * i] = q_live ? v.x : 0.0f;
            qv[4 * i + 1] = q_live ? v.y : 0.0f;
            qv[4 * i + 2] = q_live ? v.z : 0.0f;
            qv[4 * i + 3] = q_live ? v.w : 0.0f;
        }
    }
    const int wave_last = p0 + min(n, hw * 16 + 16) - 1;  // this wave's last query position
    const bool wave_live = hw * 16 < n;

    float o[4][4];  // O^T: lane l holds dims 16 dt + 4 (l/16) + r of query l%16
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 4; r++) o[dt][r] = 0.0f;
    float m = -INFINITY, lsum = 0.0f;

    for (int c = 0; c < chunks; c++) {
        __syncthreads();  // the previous chunk is consumed
#pragma unroll
        for (int i = 0; i < kChunkBlocks; i++) {
            const int pos = (fidx & 255) >> 4, d = (fidx & 15) * 4;
            const int key = i * kBlockPos + pos;
            const bool live = c * kMmaKeys + key < key_end;
            bad_block |= live && (unsigned)ids[i] >= blocks;
            const float4 cur = pre[i];
            if constexpr (FAST) {
                const float4 v = live ? cur : make_float4(0.f, 0.f, 0.f, 0.f);
                const float x[4] = {v.x, v.y, v.z, v.w};
                if (t < 256) {  // K: [key][h | m | l], 4 dimensions
                    uint16_t t3[3][4];
#pragma unroll
                    for (int j = 0; j < 4; j++) split3(x[j], t3[0][j], t3[1][j], t3[2][j]);
                    uint16_t *kp = (uint16_t *)kt + key * kKRow + d;
#pragma unroll
                    for (int p = 0; p < 3; p++)
                        *(uint2 *)(kp + p * kHeadDim) =
                            make_uint2(t3[p][0] | (uint32_t)t3[p][1] << 16,
                                       t3[p][2] | (uint32_t)t3[p][3] << 16);
                } else {  // V transposed: [dimension][hi keys | lo keys]
                    uint16_t hi[4], lo[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) split2h(x[j], hi[j], lo[j]);
                    uint16_t *vp = (uint16_t *)vt + d * kF16Row + key;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        vp[j * kF16Row] = hi[j];
                        vp[j * kF16Row + kMmaKeys] = lo[j];
                    }
                }
            } else {
                float *dst = (t < 256 ? kt : vt) + key * kMmaRow + d;
                *(float4 *)dst = live ? cur : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        __syncthreads();
        if (c + 1 < chunks) {
#pragma unroll
            for (int b = 0; b < kChunkBlocks; b++) {
                ids[b] = next_ids[b];
                const int tb = (c + 2) * kChunkBlocks + b;
                next_ids[b] = tb < table_stride ? table[tb] : 0;
            }
            PGPU_FETCH_CHUNK();
        }
        if (!wave_live) continue;
        // The chunk's 16-key sub-blocks this wave needs (the later ones are
        // past its last query): uniform over the wave.
        const int key0 = c * kMmaKeys;
        const int last = min(wave_last, key_end - 1);
        const int nsub = last < key0 ? 0 : min(kMmaKeys / 16, (last - key0) / 16 + 1);
        if (nsub <= 0) continue;
        // Scores of the whole chunk first (nsub x 16 MFMAs in four
        // independent chains per sub-block), then one softmax step for the
        // chunk, then the value sums (four independent chains, one per
        // 16-dimension tile).
        float sc[4][4];
        float bm = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 4; sub++) {
            if (sub >= nsub) {
#pragma unroll
                for (int r = 0; r < 4; r++) sc[sub][r] = -INFINITY;
                continue;
            }
            f32x4 sp[4];
#pragma unroll
            for (int u = 0; u < 4; u++) sp[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            if constexpr (FAST) {
                const uint16_t *krow =
                    (const uint16_t *)kt + (sub * 16 + (lane & 15)) * kKRow + 8 * g;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    bf16x8 k3[3];
#pragma unroll
                    for (int p = 0; p < 3; p++)
                        k3[p] = *(const bf16x8 *)(krow + p * kHeadDim + 32 * h);
                    // Smallest products first: m.m, l.h, h.l, m.h, h.m, h.h.
                    f32x4 &c = sp[h];
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3[1], q3[1][h], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3[2], q3[0][h], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3[0], q3[2][h], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3[1], q3[0][h], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3[0], q3[1][h], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k3[0], q3[0][h], c, 0, 0, 0);
                }
            } else {
                const float *krow = kt + (sub * 16 + (lane & 15)) * kMmaRow + 16 * g;
                float kk[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 v = *(const float4 *)(krow + 4 * i);
                    kk[4 * i] = v.x;
                    kk[4 * i + 1] = v.y;
                    kk[4 * i + 2] = v.z;
                    kk[4 * i + 3] = v.w;
                }
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        sp[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[4 * i + u],
                                                                     qv[4 * i + u], sp[u], 0, 0,
                                                                     0);
            }
            // Keys key0 + 16 sub + 4g + r against query qpos.
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // (FAST: sp[2], sp[3] are zero; adding them is exact.)
                const float st = __fadd_rn(__fadd_rn(sp[0][r], sp[1][r]),
                                           __fadd_rn(sp[2][r], sp[3][r]));
                const int kp = key0 + sub * 16 + 4 * g + r;
                sc[sub][r] = q_live && kp <= qpos ? st : -INFINITY;
                bm = fmaxf(bm, sc[sub][r]);
            }
        }
        bm = xor16_32_max(bm);
        const float mn = fmaxf(m, bm);
        float ps = 0.0f;
#pragma unroll
        for (int sub = 0; sub < 4; sub++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // FAST: the hardware exp2 of (s - max) * log2(e) (within
                // 2e-6 relative at |s - max| < 50, like the scores' own error).
                const float z = sc[sub][r] - mn;
                sc[sub][r] = sc[sub][r] == -INFINITY ? 0.0f : FAST ? __expf(z) : expf(z);
                ps += sc[sub][r];
            }
        ps = xor16_32_sum(ps);
        const float keep = mn == -INFINITY ? 1.0f : FAST ? __expf(m - mn) : expf(m - mn);
        m = mn;
        lsum = fmaf(lsum, keep, ps);
        f32x4 acc[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            acc[dt] = f32x4{o[dt][0] * keep, o[dt][1] * keep, o[dt][2] * keep, o[dt][3] * keep};
        if constexpr (FAST) {
#pragma unroll
            for (int p2 = 0; p2 < 2; p2++) {
                if (2 * p2 >= nsub) break;
                // P^T: slots 0-3 keys 32 p2 + 4g + r, slots 4-7 keys 32 p2 + 16 + 4g + r.
                f16x8 ph, pl;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float x = sc[2 * p2 + (j >> 2)][j & 3] * kPScale;
                    const _Float16 hi = (_Float16)x;
                    ph[j] = hi;
                    pl[j] = (_Float16)__fsub_rn(x, (float)hi);
                }
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    const uint16_t *vrow = (const uint16_t *)vt +
                                           (16 * dt + (lane & 15)) * kF16Row + 32 * p2 + 4 * g;
                    const f16x8 vh =
                        f16x8_of(*(const uint2 *)vrow, *(const uint2 *)(vrow + 16));
                    const f16x8 vl = f16x8_of(*(const uint2 *)(vrow + kMmaKeys),
                                              *(const uint2 *)(vrow + kMmaKeys + 16));
                    acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, acc[dt], 0, 0, 0);
                    acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, acc[dt], 0, 0, 0);
                    acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, acc[dt], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int sub = 0; sub < 4; sub++) {
                if (sub >= nsub) break;
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
#pragma unroll
                    for (int dt = 0; dt < 4; dt++) {
                        const float va =
                            vt[(sub * 16 + 4 * g + jj) * kMmaRow + 16 * dt + (lane & 15)];
                        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(va, sc[sub][jj], acc[dt],
                                                                       0, 0, 0);
                    }
            }
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++) o[dt][r] = acc[dt][r];
    }
#undef PGPU_FETCH_CHUNK
    if (bad_block) atomicOr(status, 2);
    if (!q_live) return;
    // Lane l holds O^T rows 16 dt + 4g .. +3 of query qi: four consecutive
    // columns of its attention row.
    const bool ok = lsum > 0.0f && isfinite(lsum);
    const float inv = 1.0f / lsum;
    bool bad = !ok;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            // FAST: o carries the 2^12 of P (taking it out is exact).
            const float acc = FAST ? o[dt][r] * (1.0f / kPScale) : o[dt][r];
            v[r] = ok ? acc * inv : 0.0f;
            bad |= !isfinite(v[r]);
        }
        if (terms == kF16Pair)
            store_split4<true>(out_split, s0 + qi, head * kHeadDim + 16 * dt + 4 * g,
                               kWidth / 32, v, false);
        else
            store_split4(out_split, s0 + qi, head * kHeadDim + 16 * dt + 4 * g, kWidth / 32, v,
                         false, terms);
    }
    flag_nonfinite(status, bad);
}

// ---------------------------------------------------------------------------
template <int EPI, bool SCALED, int WR, int WP, int RW, int PW, int NB, int KS, int FORMAT>
int launch_format(const GemmArgs &a, hipStream_t stream) {
    constexpr int RT = WR * RW, PT = WP * PW;
    const int row_groups = (a.n_rows / 16) / RT;
    const int pos_groups = ((a.streams + 15) / 16 + PT - 1) / PT;
    hipLaunchKernelGGL((k_prefill_gemm<EPI, SCALED, WR, WP, RW, PW, NB, KS, FORMAT>),
                       dim3(row_groups * pos_groups), dim3(kTaskThreads), 0, stream, a,
                       row_groups, pos_groups);
    return launch_ok("pgpu_prefill_gemm");
}

template <int EPI, bool SCALED, int WR, int WP, int RW, int PW, int NB, int KS>
int launch_gemm(const GemmArgs &a, hipStream_t stream) {
    if (a.split_terms == 2)
        return launch_format<EPI, SCALED, WR, WP, RW, PW, NB, KS, 2>(a, stream);
    return launch_format<EPI, SCALED, WR, WP, RW, PW, NB, KS, 3>(a, stream);
}

// Tile shapes (rows x positions per work-group), chosen by measurement on
// MI355X (4096 positions).
// Three split terms:
//  - MLP in (2048 rows, K = 512): 256 x 128, waves of 4 x 4 tiles, a 3 x 1
//    ring (126 KB of LDS, 256 work-groups, one per CU): 37.6 us against
//    39.5 for 128 x 64 tiles two per CU (2 x 2 tiles per wave).
//  - QKV (1536 rows): 192 x 128 (3 x 4 tiles per wave, 256 work-groups):
//    32.2 against 32.8 us.
//    With more than 4 tiles per wave the epilogue operands are loaded after
//    the main loop. A software-pipelined loop (a wave's LDS reads of block
//    k + 1 in flight during block k's MFMAs, two register sets of 4 x 2
//    tiles) was slower for every shape: 34.1-47.6 against 13.8-37.9 us.
//  - 512 rows (out, MLP out): 128 x 64 with a 2 x 2 ring (256 work-groups,
//    one per CU): 13.8 / 37.1 us; deeper rings (3 x 2, 4 x 1 .. 8 x 1) and
//    64-row or 32-position tiles were slower (two terms).
// fp16 pairs (a stage holds two thirds of the operand bytes), swept over
// six shapes per projection, ms per 16 x 256 set with the others fixed:
//  - 512 rows: 128 x 64 with a 3 x 2 ring (1.606 against 1.701 for 2 x 2);
//  - QKV: 192 x 64, 3 x 1 ring (1.651 against 1.717 for 192 x 128);
//  - MLP in: 256 x 128 with a 2 x 2 ring (1.541 against 1.552 for 3 x 1,
//    with the two above).
// A short prompt (at most kShortPrefillTiles 16-position tiles) takes
// 64 x 32 tiles, one MFMA tile per wave, so that its projections still
// spread over the CUs (a 256-position prompt: 64-256 work-groups instead
// of 16-32; a work-group's time hardly depends on its tile's size here),
// and stages of 4 blocks (8 at K = 2048, two stages in the ring): a stage
// costs a barrier and a copy wait whatever its size. Measured on the B=1
// workload's 256-position prefill, 12 layers: 1.18 ms with the large tiles,
// 0.81 with 64 x 32 tiles and 1-block stages, 0.73 with 4-block stages at
// K = 2048, 0.70 as chosen.
constexpr int kShortPrefillTiles = 32;

template <int EPI, bool SCALED>
int dispatch_gemm(const GemmArgs &a, hipStream_t stream) {
    if (a.split_terms == kF16Pair) {
        if ((a.streams + 15) / 16 <= kShortPrefillTiles) {
            if constexpr (EPI == EPI_RESIDUAL)
                if (a.k_cols == kFfn)
                    return launch_format<EPI, SCALED, 4, 2, 1, 1, 2, 8, kF16Pair>(a, stream);
            return launch_format<EPI, SCALED, 4, 2, 1, 1, 3, 4, kF16Pair>(a, stream);
        }
        if constexpr (EPI == EPI_GELU_SPLIT)
            if (a.n_rows % (8 * 256) == 0)
                return launch_format<EPI, SCALED, 4, 2, 4, 4, 2, 2, kF16Pair>(a, stream);
        if constexpr (EPI == EPI_QKV)
            if (a.n_rows % (8 * 192) == 0)
                return launch_format<EPI, SCALED, 4, 2, 3, 2, 3, 1, kF16Pair>(a, stream);
        return launch_format<EPI, SCALED, 4, 2, 2, 2, 3, 2, kF16Pair>(a, stream);
    }
    if constexpr (EPI == EPI_GELU_SPLIT)
        if (a.n_rows % (8 * 256) == 0) return launch_gemm<EPI, SCALED, 4, 2, 4, 4, 3, 1>(a, stream);
    if constexpr (EPI == EPI_QKV)
        if (a.n_rows % (8 * 192) == 0) return launch_gemm<EPI, SCALED, 4, 2, 3, 4, 3, 1>(a, stream);
    if (a.n_rows > kWidth) return launch_gemm<EPI, SCALED, 4, 2, 2, 2, 3, 1>(a, stream);
    return launch_gemm<EPI, SCALED, 4, 2, 2, 2, 2, 2>(a, stream);
}

template <int EPI>
int run_gemm(const GemmArgs &a, const pgpu_wide_matrix *w, hipStream_t stream) {
    if (!w || !w->values || a.n_rows % 128 || (a.k_cols != kWidth && a.k_cols != kFfn) ||
        a.streams <= 0 || !a.xs || !a.status ||
        (a.split_terms != 2 && a.split_terms != 3 && a.split_terms != kF16Pair) ||
        (a.split_terms == kF16Pair && !w->values_f16))
        return bad_arguments("pgpu_prefill_gemm");
    return w->scales ? dispatch_gemm<EPI, true>(a, stream) : dispatch_gemm<EPI, false>(a, stream);
}

GemmArgs gemm_args(const pgpu_wide_matrix *w, const uint16_t *split, int streams, int terms,
                   int *status) {
    GemmArgs a{};
    a.split_terms = terms;
    if (!w) return a;
    a.xs = split;
    a.w = terms == kF16Pair ? w->values_f16 : w->values;
    a.wscale_f = w->scales;
    a.n_rows = (int)w->rows;
    a.k_cols = (int)w->columns;
    a.streams = streams;
    a.status = status;
    return a;
}

}  // namespace
}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_rows_split_ln(void *stream, const float *rows, const float *weight,
                                  const float *bias, float epsilon, int streams, int terms,
                                  uint16_t *out_split, int *status) {
    if (!rows || !weight || !bias || !out_split || !status || streams <= 0 ||
        !(epsilon > 0.0f) || terms < 1 || terms > kF16Pair)
        return bad_arguments("pgpu_rows_split_ln");
    // Whole 16-row tiles: the rows past `streams` are written as zeros.
    const int tiles = (streams + 15) / 16;
    hipLaunchKernelGGL(k_rows_split_ln, dim3(tiles), dim3(512), 0, (hipStream_t)stream, rows,
                       weight, bias, epsilon, streams, terms, out_split, status);
    return launch_ok("pgpu_rows_split_ln");
}

extern "C" int pgpu_rows_split_attention(void *stream, const pgpu_attention_scratch *work,
                                         const int32_t *positions, int streams, int max_splits,
                                         uint16_t *out_split, int *status) {
    if (!work || !positions || !out_split || !status || streams <= 0 ||
        streams > work->max_streams || max_splits <= 0 || max_splits > work->max_splits)
        return bad_arguments("pgpu_rows_split_attention");
    GemmArgs a{};
    a.part_acc = work->part_acc;
    a.part_ml = work->part_ml;
    a.max_splits = max_splits;
    a.positions = positions;
    a.streams = streams;
    a.status = status;
    hipLaunchKernelGGL(k_rows_split<SRC_ATTN>, dim3((streams + 15) / 16), dim3(kTaskThreads), 0,
                       (hipStream_t)stream, a, out_split);
    return launch_ok("pgpu_rows_split_attention");
}

extern "C" int pgpu_prefill_gemm_qkv(void *stream, const pgpu_wide_matrix *w, const uint16_t *split,
                                     int streams, int terms, const pgpu_paged_kv *kv, int layer,
                                     const int32_t *tables, int table_stride,
                                     const int32_t *positions, const float *rope, float *q_out,
                                     int *status) {
    if (!w || w->rows != 3 * kWidth || w->columns != kWidth || !kv || layer < 0 ||
        layer >= kv->layers || !tables || table_stride <= 0 || !positions || !rope || !q_out)
        return bad_arguments("pgpu_prefill_gemm_qkv");
    GemmArgs a = gemm_args(w, split, streams, terms, status);
    a.q_out = q_out;
    a.kv = kv->base;
    a.layer_stride = kv->layer_stride;
    a.blocks = (unsigned)kv->blocks;
    a.layer = layer;
    a.tables = tables;
    a.table_stride = table_stride;
    a.positions = positions;
    a.rope = (const float2 *)rope;
    a.plain_qkv = true;  // read by the next launches only
    return run_gemm<EPI_QKV>(a, w, (hipStream_t)stream);
}

extern "C" int pgpu_prefill_gemm_residual(void *stream, const pgpu_wide_matrix *w,
                                          const uint16_t *split, int streams, int terms,
                                          const float *residual, float *out, int *status) {
    if (!w || !residual || !out) return bad_arguments("pgpu_prefill_gemm_residual");
    GemmArgs a = gemm_args(w, split, streams, terms, status);
    a.out = out;
    a.ld_out = (int)w->rows;
    a.residual = residual;
    return run_gemm<EPI_RESIDUAL>(a, w, (hipStream_t)stream);
}

extern "C" int pgpu_prefill_gemm_gelu_split(void *stream, const pgpu_wide_matrix *w,
                                            const uint16_t *split, int streams, int terms,
                                            uint16_t *out_split, int *status) {
    if (!w || !out_split || w->rows % 32) return bad_arguments("pgpu_prefill_gemm_gelu_split");
    GemmArgs a = gemm_args(w, split, streams, terms, status);
    a.out_split = out_split;
    a.out_kb = (int)w->rows / 32;
    a.out_terms = terms;  // the MLP-out projection reads as many terms
    return run_gemm<EPI_GELU_SPLIT>(a, w, (hipStream_t)stream);
}

extern "C" int pgpu_prefill_attention_rows(void *stream, const float *q, const pgpu_paged_kv *kv,
                                           int layer, const int32_t *tables, int table_stride,
                                           const int32_t *positions, int streams,
                                           const int32_t *entries, int entry_count,
                                           uint16_t *out_split, int terms, int *status) {
    if (!q || !kv || !tables || !positions || !entries || !out_split || !status ||
        streams <= 0 || layer < 0 || layer >= kv->layers || table_stride <= 0 ||
        entry_count <= 0 || entry_count > 65535 || terms < 2 || terms > kF16Pair)
        return bad_arguments("pgpu_prefill_attention_rows");
    hipLaunchKernelGGL(k_prefill_attention_rows, dim3(entry_count, kHeads),
                       dim3(64 * kAttnWaves), 0, (hipStream_t)stream, q, kv->base,
                       kv->layer_stride, (unsigned)kv->blocks, layer, tables, table_stride,
                       positions, streams, entries, out_split, terms, status);
    return launch_ok("pgpu_prefill_attention_rows");
}

extern "C" int pgpu_prefill_attention_mfma(void *stream, const float *q, const pgpu_paged_kv *kv,
                                           int layer, const int32_t *tables, int table_stride,
                                           const int32_t *positions, int streams,
                                           const int32_t *pairs, int pair_count,
                                           uint16_t *out_split, int terms, int *status) {
    if (!q || !kv || !tables || !positions || !pairs || !out_split || !status ||
        streams <= 0 || layer < 0 || layer >= kv->layers || table_stride <= 0 ||
        pair_count <= 0 || pair_count > 65535 || terms < 2 || terms > kF16Pair)
        return bad_arguments("pgpu_prefill_attention_mfma");
    const dim3 grid(pair_count, kHeads), block(kPairThreads);
    if (terms == kF16Pair)
        hipLaunchKernelGGL(k_prefill_attention_mfma<true>, grid, block, 0, (hipStream_t)stream, q,
                           kv->base, kv->layer_stride, (unsigned)kv->blocks, layer, tables,
                           table_stride, positions, streams, pairs, out_split, terms, status);
    else
        hipLaunchKernelGGL(k_prefill_attention_mfma<false>, grid, block, 0, (hipStream_t)stream,
                           q, kv->base, kv->layer_stride, (unsigned)kv->blocks, layer, tables,
                           table_stride, positions, streams, pairs, out_split, terms, status);
    return launch_ok("pgpu_prefill_attention_mfma");
}

extern "C" int pgpu_wide_from_matrix(void *stream, const pgpu_matrix *w, uint16_t *values,
                                     float *scales, uint16_t *values_f16) {
    if (!w || !w->q8 || !w->values || !w->scales || !values || !scales || w->rows % 16 ||
        w->columns % 32)
        return bad_arguments("pgpu_wide_from_matrix");
    const size_t n = w->rows * w->columns;
    const unsigned blocks = (unsigned)((n / 8 + 255) / 256 < 2048 ? (n / 8 + 255) / 256 : 2048);
    hipLaunchKernelGGL(k_wide_from_q8, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       (const int8_t *)w->values, w->scales, n, values, scales, values_f16);
    return launch_ok("pgpu_wide_from_matrix");
}
