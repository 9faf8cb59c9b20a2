// Single-query causal attention over a paged fp32 KV pool, split over keys.
//
// Replaces flow_attention (src/phonon_transformer.c:338-404), called per head
// by phonon_flow_layer_step (src/phonon_transformer.c:429-435). Softmax is
// online: the reference uses 512-key blocks, this kernel 64-key wave blocks
// merged in fixed order; results agree to fp32 rounding (tolerance-checked).
//
// Pool layout, per layer: [block][head][K|V][16 positions][64] fp32, so one
// (block, head) tile of keys is 4 KB contiguous and its values follow it.
// Split unit (head h, split j, stream s) = 8 waves covering keys
// [256j, 256j+256) of stream s: wave w takes blocks 16j+2w, 16j+2w+1. Each
// lane loads float4s at tile offsets 256*i + 4*lane (i = 0..3), i.e. key
// 4i + lane/16, dims 4*(lane%16) .. +3: every load instruction reads 1 KB
// contiguous, and all 16 loads of a wave are in flight together.
//
// Each work-group writes its split's (max, sum, unnormalised P.V) partial;
// the splits are merged by whoever consumes the output (the out-projection
// prologue in the decode step, or k_attention_merge). There is no
// cross-work-group handshake: on gfx950 an agent-scope fence writes back and
// invalidates the whole L2 and costs far more than a separate merge.
#include "pgpu_common.hpp"
#include "phonon_gpu.h"

namespace pgpu {

struct AttnArgs {
    const float *q;           // [streams][512], RoPE'd, scaled by 1/8
    const float *kv;
    size_t layer_stride;
    unsigned blocks;          // blocks per layer; table entries must be below
    int layer;
    const int32_t *tables;
    int table_stride;
    const int32_t *positions; // keys attended = positions[s] + 1
    int streams, max_splits;
    float *part_acc;          // [streams*8*max_splits][64]
    float *part_ml;           // [streams*8*max_splits][2]
    int *status;
};



// K/V bytes are read once per step: non-temporal loads, so the stream does
// not displace what the other kernels of the step re-read from the caches
// (projection weights, activations).
__device__ inline float4 stream_load(const float *p) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_nontemporal_load((const f4 *)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// Waves per split unit and K/V blocks per wave: a unit of 8 waves x 2 blocks
// covers one 256-key split; each wave keeps its 16 float4 of K/V in
// flight at once (64 registers), so a 1024-thread work-group (2 units) stays
// within 128 registers per lane.
constexpr int kUnitWaves = 8, kBlocksPerWave = 2;

struct AttnShared {
    float4 acc[kUnitWaves][16];
    float m[kUnitWaves], l[kUnitWaves];
};

// Split `split` of head `head` of stream `s`, by the unit's 8 waves (`wave`
// = 0..7 within the unit). Every wave of the work-group must call it (it
// holds one work-group barrier); a unit without live keys only takes part
// in the barrier. Writes the split's (max, sum, unnormalised P.V) partial.
__device__ inline void attend_split(const AttnArgs &a, int head, int split, int s, int wave,
                                    AttnShared &sh) {
    const int lane = threadIdx.x & 63;
    const int krow = lane >> 4, dcol = lane & 15;
    const int count = a.positions[s] + 1;
    const int nsplit = (count + kSplitKeys - 1) / kSplitKeys;
    // A context the grid or the block table cannot cover is an error, never
    // a partial read: flag it once, and the unit computes nothing.
    const bool covered =
        count >= 1 && nsplit <= a.max_splits && count <= a.table_stride * kBlockPos;
    if (!covered && split == 0 && wave == 0 && lane == 0) atomicOr(a.status, 2);
    const bool live = covered && split * kSplitKeys < count;  // uniform per unit

    float m = -INFINITY, l = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
        const float4 q = *(const float4 *)(a.q + (size_t)s * kWidth + head * kHeadDim + dcol * 4);
        const int32_t *__restrict__ table = a.tables + (size_t)s * a.table_stride;
        const float *layer_kv = a.kv + (size_t)a.layer * a.layer_stride;
        const int first_block = split * 16 + wave * kBlocksPerWave;
        const int stream_blocks = (count + kBlockPos - 1) / kBlockPos;
        // < first_block: this wave has no keys
        const int last_block = min(first_block + kBlocksPerWave - 1, stream_blocks - 1);

        // Block ids first (uniform), then every K/V load of the wave at once.
        // Blocks past the context re-read the last valid block (their keys
        // are masked below); an id outside the pool is flagged and replaced.
        int ids[kBlocksPerWave];
        bool bad_block = false;
#pragma unroll
        for (int t = 0; t < kBlocksPerWave; t++) {
            const int b = min(first_block + t, max(last_block, first_block));
            const int id = last_block >= first_block ? table[b] : 0;
            bad_block |= (unsigned)id >= a.blocks;
            ids[t] = (unsigned)id < a.blocks ? id : 0;
        }
        float4 kr[kBlocksPerWave][4], vr[kBlocksPerWave][4];
        if (last_block >= first_block) {
#pragma unroll
            for (int t = 0; t < kBlocksPerWave; t++) {
                const float *tile =
                    layer_kv + ((size_t)ids[t] * kHeads + head) * 2048 + lane * 4;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    kr[t][i] = stream_load(tile + i * 256);
                    vr[t][i] = stream_load(tile + 1024 + i * 256);
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < kBlocksPerWave; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    kr[t][i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    vr[t][i] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
        }
        if (bad_block && lane == 0) atomicOr(a.status, 2);

        float score[kBlocksPerWave][4];
#pragma unroll
        for (int t = 0; t < kBlocksPerWave; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 k = kr[t][i];
                float d = q.x * k.x;
                d = fmaf(q.y, k.y, d);
                d = fmaf(q.z, k.z, d);
                d = fmaf(q.w, k.w, d);
                d = row16_sum(d);
                const int key = (first_block + t) * kBlockPos + i * 4 + krow;
                score[t][i] = key < count ? d : -INFINITY;
                m = fmaxf(m, score[t][i]);
            }
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
#pragma unroll
        for (int t = 0; t < kBlocksPerWave; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // Slots past the context hold whatever the pool held before:
                // they are skipped, never multiplied by a zero weight.
                if (score[t][i] == -INFINITY) continue;
                const float e = expf(score[t][i] - m);
                l += e;
                acc.x = fmaf(e, vr[t][i].x, acc.x);
                acc.y = fmaf(e, vr[t][i].y, acc.y);
                acc.z = fmaf(e, vr[t][i].z, acc.z);
                acc.w = fmaf(e, vr[t][i].w, acc.w);
            }
        // Lanes of one key row hold the same l; sum the four rows.
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        acc.x += __shfl_xor(acc.x, 16);
        acc.y += __shfl_xor(acc.y, 16);
        acc.z += __shfl_xor(acc.z, 16);
        acc.w += __shfl_xor(acc.w, 16);
        acc.x += __shfl_xor(acc.x, 32);
        acc.y += __shfl_xor(acc.y, 32);
        acc.z += __shfl_xor(acc.z, 32);
        acc.w += __shfl_xor(acc.w, 32);
        if (lane < 16) sh.acc[wave][lane] = acc;
        if (lane == 0) {
            sh.m[wave] = m;
            sh.l[wave] = l;
        }
    }
    __syncthreads();
    if (!live || wave != 0 || lane >= 16) return;

    // Merge the unit's waves (fixed order). A wave without keys has l = 0.
    float mm = sh.m[0];
#pragma unroll
    for (int w = 1; w < kUnitWaves; w++) mm = fmaxf(mm, sh.m[w]);
    float ll = 0.0f;
    float4 aa = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < kUnitWaves; w++) {
        if (sh.l[w] == 0.0f) continue;
        const float f = expf(sh.m[w] - mm);
        ll = fmaf(sh.l[w], f, ll);
        const float4 x = sh.acc[w][lane];
        aa.x = fmaf(x.x, f, aa.x);
        aa.y = fmaf(x.y, f, aa.y);
        aa.z = fmaf(x.z, f, aa.z);
        aa.w = fmaf(x.w, f, aa.w);
    }
    const size_t slot = ((size_t)s * kHeads + head) * a.max_splits + split;
    *(float4 *)(a.part_acc + slot * 64 + lane * 4) = aa;
    if (lane == 0) *(float2 *)(a.part_ml + slot * 2) = make_float2(mm, ll);
}

// One split unit per 512-thread work-group. Heads vary fastest across the
// grid: work-groups dispatched together read all 8 heads' tiles of the same
// blocks (64 KB contiguous each).
__global__ __launch_bounds__(64 * kUnitWaves) void k_attention(AttnArgs a) {
    __shared__ AttnShared sh;
    // The wave index is uniform: readfirstlane lets the block ids come from
    // scalar loads, so no vector-load wait sits between the K/V loads.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    attend_split(a, blockIdx.x, blockIdx.y, blockIdx.z, wave, sh);
}

// Merge of the split partials into fp32 rows and/or split fragments, one
// wave per (head, stream): lane d produces dimension d.
__global__ __launch_bounds__(64) void k_attention_merge(const float *__restrict__ part_acc,
                                                        const float *__restrict__ part_ml,
                                                        const int32_t *__restrict__ positions,
                                                        int max_splits, float *out,
                                                        uint16_t *out_split, int *status) {
    const int head = blockIdx.x, s = blockIdx.y, d = threadIdx.x;
    const int count = positions[s] + 1;
    const int nsplit = min((count + kSplitKeys - 1) / kSplitKeys, max_splits);
    const size_t first = ((size_t)s * kHeads + head) * max_splits;
    float mx = -INFINITY;
    for (int j = 0; j < nsplit; j++) mx = fmaxf(mx, part_ml[(first + j) * 2]);
    float total = 0.0f, acc = 0.0f;
    for (int j = 0; j < nsplit; j++) {
        const float f = expf(part_ml[(first + j) * 2] - mx);
        total = fmaf(part_ml[(first + j) * 2 + 1], f, total);
        acc = fmaf(part_acc[(first + j) * 64 + d], f, acc);
    }
    const float o = acc * (1.0f / total);
    const bool bad = !(total > 0.0f) || !isfinite(total) || !isfinite(o);
    const int col = head * kHeadDim + d;
    if (out) out[(size_t)s * kWidth + col] = o;
    if (out_split) {
        uint16_t h, m, l;
        split3(o, h, m, l);
        const size_t base = split_index(s, col, 0, kWidth / 32);
        out_split[base] = h;
        out_split[base + 512] = m;
        out_split[base + 1024] = l;
    }
    flag_nonfinite(status, bad);
}

}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_attention(void *stream, const float *q, const pgpu_paged_kv *kv, int layer,
                              const int32_t *tables, int table_stride, const int32_t *positions,
                              int streams, int heads, int max_splits,
                              const pgpu_attention_scratch *scratch, int *status) {
    if (streams <= 0 || heads <= 0 || heads > kHeads || max_splits <= 0 || layer < 0 ||
        layer >= kv->layers || max_splits > scratch->max_splits ||
        streams > scratch->max_streams)
        return bad_arguments("pgpu_attention");
    AttnArgs a;
    a.q = q;
    a.kv = kv->base;
    a.layer_stride = kv->layer_stride;
    a.blocks = (unsigned)kv->blocks;
    a.layer = layer;
    a.tables = tables;
    a.table_stride = table_stride;
    a.positions = positions;
    a.streams = streams;
    a.max_splits = max_splits;
    a.part_acc = scratch->part_acc;
    a.part_ml = scratch->part_ml;
    a.status = status;
    hipLaunchKernelGGL(k_attention, dim3(heads, max_splits, streams), dim3(64 * kUnitWaves), 0,
                       (hipStream_t)stream, a);
    return launch_ok("pgpu_attention");
}

extern "C" int pgpu_attention_merge(void *stream, const pgpu_attention_scratch *scratch,
                                    const int32_t *positions, int streams, int heads,
                                    int max_splits, float *out, uint16_t *out_split,
                                    int *status) {
    if (streams <= 0 || heads <= 0 || heads > kHeads || max_splits <= 0 ||
        max_splits > scratch->max_splits || streams > scratch->max_streams ||
        (!out && !out_split))
        return bad_arguments("pgpu_attention_merge");
    hipLaunchKernelGGL(k_attention_merge, dim3(heads, streams), dim3(64), 0,
                       (hipStream_t)stream, scratch->part_acc, scratch->part_ml, positions,
                       max_splits, out, out_split, status);
    return launch_ok("pgpu_attention_merge");
}
