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
#include <mutex>

#include "pgpu_attention.hpp"
#include "pgpu_common.hpp"
#include "phonon_gpu.h"

// Split partials of pgpu_attention_static: a fixed device array instead of a
// caller's pgpu_attention_scratch, so that the entry point allocates
// nothing. Slots [0, kStaticSlots) of 64 floats (unnormalised P.V), then
// kStaticSlots (max, sum) pairs. Every device holds its own copy until the
// process ends; host code uses its per-device address (from
// pgpu_attention_static_setup), never the array's name.
constexpr int kStaticSlots = PGPU_ATTENTION_STATIC_SLOTS;
static __device__ __align__(256) float scratch[(size_t)kStaticSlots * (64 + 2)];

namespace pgpu {

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

// Causal attention of a batched prefill. A work entry (s0, s1, split) names
// consecutive positions of one stream: pseudo-streams s0 .. s1-1 (at most
// kPrefillQueries), which share that stream's block table row. One
// work-group per (head, entry) loads the split's K/V tile once, the 8 waves
// x 2 blocks of a split unit, into registers (up to the context of the
// entry's last query), then walks the queries: for each query whose context
// reaches the split it computes the split's partial with exactly the
// arithmetic of attend_unit (same key order, masking, row sums, exp,
// fused multiply-adds and wave merge), so a prefill gives the bits of
// decoding the same positions one step at a time. A stream's K/V are read
// once per entry instead of once per position.
constexpr int kPrefillQueries = 64;  // queries per entry (host-enforced)
constexpr int kPrefillBatch = 8;     // queries whose wave partials share one LDS round

__global__ __launch_bounds__(64 * kUnitWaves) void k_prefill_attention(AttnArgs a,
                                                                       const int4 *entries) {
    __shared__ AttnShared sh[kPrefillBatch];
    const int head = blockIdx.x;
    const int4 e = entries[blockIdx.y];
    // An entry outside the streams or the partial layout is an error: the
    // work-group writes nothing (the host builds valid entries).
    if (e.x < 0 || e.y > a.streams || e.y <= e.x || e.y - e.x > kPrefillQueries || e.z < 0 ||
        e.z >= a.max_splits) {
        if (threadIdx.x == 0) atomicOr(a.status, 2);
        return;
    }
    const int s0 = e.x, nq = e.y - e.x, split = e.z;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, krow = lane >> 4, dcol = lane & 15;
    // Lane i holds the position of query s0 + i; the tile is loaded up to
    // the context of the entry's latest query.
    const int my_pos = lane < nq ? a.positions[s0 + lane] : -1;
    int top = my_pos;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) top = max(top, __shfl_xor(top, o));
    const int32_t *__restrict__ table = a.tables + (size_t)s0 * a.table_stride;
    const int top_blocks = min((top + kBlockPos) / kBlockPos, a.table_stride);
    const float *layer_kv = a.kv + (size_t)a.layer * a.layer_stride;
    bool bad_block = false;
    float4 kr[kBlocksPerWave][4], vr[kBlocksPerWave][4];
#pragma unroll
    for (int t = 0; t < kBlocksPerWave; t++) {
        const int b = split * 16 + wave * kBlocksPerWave + t;
        if (b < top_blocks) {  // uniform
            const int raw = table[b];
            bad_block |= (unsigned)raw >= a.blocks;
            const int id = (unsigned)raw < a.blocks ? raw : 0;
            const float *tile = layer_kv + ((size_t)id * kHeads + head) * 2048 + lane * 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[t][i] = stream_load(tile + i * 256);
                vr[t][i] = stream_load(tile + 1024 + i * 256);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[t][i] = make_float4(0.f, 0.f, 0.f, 0.f);
                vr[t][i] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    }
    if (bad_block && lane == 0) atomicOr(a.status, 2);

    for (int q0 = 0; q0 < nq; q0 += kPrefillBatch) {
        const int nb = min(kPrefillBatch, nq - q0);
        // This batch's q rows, requested together.
        float4 qv[kPrefillBatch];
#pragma unroll
        for (int u = 0; u < kPrefillBatch; u++) {
            const int s = s0 + q0 + min(u, nb - 1);
            qv[u] = *(const float4 *)(a.q + (size_t)s * kWidth + head * kHeadDim + dcol * 4);
        }
#pragma unroll
        for (int u = 0; u < kPrefillBatch; u++) {
            if (u >= nb) break;
            const int count = __shfl(my_pos, q0 + u) + 1;  // uniform
            const int nsplit = (count + kSplitKeys - 1) / kSplitKeys;
            const bool covered =
                count >= 1 && nsplit <= a.max_splits && count <= a.table_stride * kBlockPos;
            if (!covered && split == 0 && wave == 0 && lane == 0) atomicOr(a.status, 2);
            if (!(covered && split * kSplitKeys < count)) continue;  // uniform
            const int first_block = split * 16 + wave * kBlocksPerWave;
            const float4 q = qv[u];
            float m = -INFINITY, l = 0.0f;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
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
            m = xor16_32_max(m);
#pragma unroll
            for (int t = 0; t < kBlocksPerWave; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (score[t][i] == -INFINITY) continue;
                    const float ex = expf(score[t][i] - m);
                    l += ex;
                    acc.x = fmaf(ex, vr[t][i].x, acc.x);
                    acc.y = fmaf(ex, vr[t][i].y, acc.y);
                    acc.z = fmaf(ex, vr[t][i].z, acc.z);
                    acc.w = fmaf(ex, vr[t][i].w, acc.w);
                }
            l = xor16_32_sum(l);
            acc.x = xor16_32_sum(acc.x);
            acc.y = xor16_32_sum(acc.y);
            acc.z = xor16_32_sum(acc.z);
            acc.w = xor16_32_sum(acc.w);
            if (lane < 16) sh[u].acc[wave][lane] = acc;
            if (lane == 0) {
                sh[u].m[wave] = m;
                sh[u].l[wave] = l;
            }
        }
        __syncthreads();
        // Wave w merges query q0 + w of the batch, in fixed wave order (the
        // position is read by every lane, before the branch).
        const int merge_pos = __shfl(my_pos, q0 + min(wave, nb - 1));
        if (wave < nb && lane < 16) {
            const int count = merge_pos + 1;
            const int nsplit = (count + kSplitKeys - 1) / kSplitKeys;
            const bool covered =
                count >= 1 && nsplit <= a.max_splits && count <= a.table_stride * kBlockPos;
            if (covered && split * kSplitKeys < count) {
                const AttnShared &r = sh[wave];
                float mx = r.m[0];
#pragma unroll
                for (int w = 1; w < kUnitWaves; w++) mx = fmaxf(mx, r.m[w]);
                float total = 0.0f;
                float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int w = 0; w < kUnitWaves; w++) {
                    if (r.l[w] == 0.0f) continue;
                    const float f = expf(r.m[w] - mx);
                    total = fmaf(r.l[w], f, total);
                    const float4 x = r.acc[w][lane];
                    o.x = fmaf(x.x, f, o.x);
                    o.y = fmaf(x.y, f, o.y);
                    o.z = fmaf(x.z, f, o.z);
                    o.w = fmaf(x.w, f, o.w);
                }
                const size_t slot =
                    ((size_t)(s0 + q0 + wave) * kHeads + head) * a.max_splits + split;
                *(float4 *)(a.part_acc + slot * 64 + lane * 4) = o;
                if (lane == 0) *(float2 *)(a.part_ml + slot * 2) = make_float2(mx, total);
            }
        }
        __syncthreads();
    }
}

}  // namespace pgpu

using namespace pgpu;

static AttnArgs attention_args(const float *q, const pgpu_paged_kv *kv, int layer,
                               const int32_t *tables, int table_stride,
                               const int32_t *positions, int streams, int max_splits,
                               float *part_acc, float *part_ml, int *status) {
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
    a.part_acc = part_acc;
    a.part_ml = part_ml;
    a.status = status;
    return a;
}

extern "C" int pgpu_attention(void *stream, const float *q, const pgpu_paged_kv *kv, int layer,
                              const int32_t *tables, int table_stride, const int32_t *positions,
                              int streams, int heads, int max_splits,
                              const pgpu_attention_scratch *work, int *status) {
    if (streams <= 0 || heads <= 0 || heads > kHeads || max_splits <= 0 || layer < 0 ||
        layer >= kv->layers || max_splits > work->max_splits || streams > work->max_streams)
        return bad_arguments("pgpu_attention");
    const AttnArgs a = attention_args(q, kv, layer, tables, table_stride, positions, streams,
                                      max_splits, work->part_acc, work->part_ml, status);
    hipLaunchKernelGGL(k_attention, dim3(heads, max_splits, streams), dim3(64 * kUnitWaves), 0,
                       (hipStream_t)stream, a);
    return launch_ok("pgpu_attention");
}

extern "C" int pgpu_attention_merge(void *stream, const pgpu_attention_scratch *work,
                                    const int32_t *positions, int streams, int heads,
                                    int max_splits, float *out, uint16_t *out_split,
                                    int *status) {
    if (streams <= 0 || heads <= 0 || heads > kHeads || max_splits <= 0 ||
        max_splits > work->max_splits || streams > work->max_streams || (!out && !out_split))
        return bad_arguments("pgpu_attention_merge");
    hipLaunchKernelGGL(k_attention_merge, dim3(heads, streams), dim3(64), 0,
                       (hipStream_t)stream, work->part_acc, work->part_ml, positions,
                       max_splits, out, out_split, status);
    return launch_ok("pgpu_attention_merge");
}

extern "C" int pgpu_prefill_attention(void *stream, const float *q, const pgpu_paged_kv *kv,
                                      int layer, const int32_t *tables, int table_stride,
                                      const int32_t *positions, int streams, int heads,
                                      int max_splits, const int32_t *entries, int entry_count,
                                      const pgpu_attention_scratch *work, int *status) {
    if (!q || !kv || !tables || !positions || !entries || !work || !status || streams <= 0 ||
        heads <= 0 || heads > kHeads || max_splits <= 0 || layer < 0 || layer >= kv->layers ||
        table_stride <= 0 || entry_count <= 0 || entry_count > 65535 ||
        max_splits > work->max_splits || streams > work->max_streams)
        return bad_arguments("pgpu_prefill_attention");
    const AttnArgs a = attention_args(q, kv, layer, tables, table_stride, positions, streams,
                                      max_splits, work->part_acc, work->part_ml, status);
    hipLaunchKernelGGL(k_prefill_attention, dim3(heads, entry_count), dim3(64 * kUnitWaves), 0,
                       (hipStream_t)stream, a, (const int4 *)entries);
    return launch_ok("pgpu_prefill_attention");
}

// --------------------------------------------------------------------------
// The static partials' device address, per device. Looked up once per device
// with that device current: by the library's init (pgpu_device_init), and by
// an entry point's first call on any other device. hipGetSymbolAddress
// allocates nothing.
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_static_lock;
float *g_static_partials[kMaxDevices];
}  // namespace

extern "C" __attribute__((visibility("hidden"))) float *pgpu_attention_static_setup(void) {
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        pgpu_record_error("pgpu_attention_static: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> hold(g_static_lock);
    if (!g_static_partials[device]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            char text[256];
            snprintf(text, sizeof(text), "pgpu_attention_static: hipGetSymbolAddress: %s",
                     hipGetErrorString(e));
            pgpu_record_error(text);
            return nullptr;
        }
        g_static_partials[device] = (float *)ptr;
    }
    return g_static_partials[device];
}

extern "C" int pgpu_attention_static(void *stream, const float *q, const pgpu_paged_kv *kv,
                                     int layer, const int32_t *tables, int table_stride,
                                     const int32_t *positions, int streams, int heads,
                                     int max_splits, float *out, uint16_t *out_split,
                                     int *status) {
    if (!q || !kv || !tables || !positions || !status || streams <= 0 || heads <= 0 ||
        heads > kHeads || max_splits <= 0 || table_stride <= 0 || layer < 0 ||
        layer >= kv->layers || (!out && !out_split))
        return bad_arguments("pgpu_attention_static");
    // The partial layout is [stream][8 heads][max_splits] whatever `heads` is.
    if ((size_t)streams * kHeads * (size_t)max_splits > (size_t)kStaticSlots) {
        char text[256];
        snprintf(text, sizeof(text),
                 "pgpu_attention_static: %d streams x %d heads x %d splits exceed the %d "
                 "partial slots of the static scratch",
                 streams, kHeads, max_splits, kStaticSlots);
        pgpu_record_error(text);
        return 0;
    }
    float *const ptr = pgpu_attention_static_setup();
    if (!ptr) return 0;
    float *const part_acc = ptr, *const part_ml = ptr + (size_t)kStaticSlots * 64;
    const AttnArgs a = attention_args(q, kv, layer, tables, table_stride, positions, streams,
                                      max_splits, part_acc, part_ml, status);
    hipLaunchKernelGGL(k_attention, dim3(heads, max_splits, streams), dim3(64 * kUnitWaves), 0,
                       (hipStream_t)stream, a);
    if (!launch_ok("pgpu_attention_static")) return 0;
    hipLaunchKernelGGL(k_attention_merge, dim3(heads, streams), dim3(64), 0,
                       (hipStream_t)stream, part_acc, part_ml, positions, max_splits, out,
                       out_split, status);
    return launch_ok("pgpu_attention_static");
}
