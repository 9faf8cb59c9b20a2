// Split-attention unit shared by the attention kernels (pgpu_attention.hip)
// and the one-launch decode step (pgpu_flow.hip). See pgpu_attention.hip for
// the pool layout and the work decomposition.
#pragma once

#include <type_traits>

#include "pgpu_common.hpp"

namespace pgpu {

struct AttnArgs {
    const float *q;           // [streams][512], RoPE'd, scaled by 1/8
    const float *kv;
    size_t layer_stride;
    unsigned blocks;          // blocks per layer; table entries must be below
    int layer;
    const int32_t *tables;
    int table_stride;
    const int32_t *positions; // keys attended = positions[s] + pos_delta + 1
    int pos_delta = 0;        // steps the stored positions trail the step's
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
// covers one 256-key split; each wave keeps its 16 float4 of K/V in flight
// at once (64 registers).
constexpr int kUnitWaves = 8, kBlocksPerWave = 2;

struct AttnShared {
    float4 acc[kUnitWaves][16];
    float m[kUnitWaves], l[kUnitWaves];
};

// What a unit found, uniform over the unit.
enum UnitState {
    UNIT_EMPTY = 0,      // the split starts past the context (or the unit does not exist)
    UNIT_LIVE = 1,       // keys attended; the partial is in wave 0
    UNIT_UNCOVERED = 2,  // the context does not fit the grid or the table (flagged)
};

// A unit's inputs gate. probe() is issued with the unit's first loads;
// pass(probe, needed) is then called by every thread before the unit reads
// anything written in the current step (the one-launch step waits there for
// the QKV tasks, unless the unit has nothing to do). NoGate: no wait.
struct NoGate {
    __device__ unsigned probe() const { return 0u; }
    __device__ void pass(unsigned, bool) const {}
};

// A gate with `kTaggedQkv` (true) hands the unit this step's q and the
// appended key's K and V itself (poll_qkv, after pass): the unit then
// requests every block, the context's last one included, before the gate,
// and replaces the appended key's slot with the handed-over K and V.
template <class G, class = void>
struct GateTaggedQkv : std::false_type {};
template <class G>
struct GateTaggedQkv<G, std::void_t<decltype(G::kTaggedQkv)>>
    : std::integral_constant<bool, G::kTaggedQkv> {};

// Splits split0 .. split0 + ROUNDS - 1 of head `head` of stream `s`, one
// after the other, by the unit's 8 waves (`wave` = 0..7 within the unit).
// Each split's partial is computed exactly as a one-round unit computes it;
// the next split's K (V) loads go out as soon as the current split's K (V)
// registers are consumed, so they overlap its softmax and wave merge. Every
// wave of the work-group must call it (it holds one work-group barrier); a
// unit without live keys (or that does not `exist`: past the end of a grid)
// only takes part in the barrier. If the result is UNIT_LIVE, lanes 0..15 of
// waves 0 .. merge_waves - 1 (each computes the same bits) hold the partial
// of each split r that starts inside the context:
// max score mm[r], sum of exp ll[r] and the unnormalised P.V dims
// [4 lane, 4 lane + 4) in aa[r]. `count` receives the stream's keys (0 if
// the unit does not exist). sh holds ROUNDS AttnShared. `rounds` (at most
// ROUNDS, uniform) limits the splits at run time. `early`: every key before
// the stream's last was written before the gate's inputs (not so in a
// batched prefill, where earlier positions append in the same launch).
template <int ROUNDS = 1, class Gate = NoGate>
__device__ inline int attend_unit(const AttnArgs &a, int head, int split0, int s, int wave,
                                  AttnShared *sh, bool exists, float4 *aa, float *mm, float *ll,
                                  int &count, const Gate &gate = Gate{}, int rounds = ROUNDS,
                                  bool early = true, int merge_waves = 1) {
    const int lane = threadIdx.x & 63;
    const int krow = lane >> 4, dcol = lane & 15;
    // First loads, in flight together: the context length, the wave's block
    // table entries (index clamped into the row; entries past the context
    // are not used) and the gate's first check.
    const int32_t *__restrict__ table = a.tables + (size_t)s * a.table_stride;
    const int position = exists ? a.positions[s] + a.pos_delta : -1;
    int ids[ROUNDS][kBlocksPerWave];
#pragma unroll
    for (int r = 0; r < ROUNDS; r++)
#pragma unroll
        for (int t = 0; t < kBlocksPerWave; t++)
            ids[r][t] = exists && r < rounds
                            ? table[min((split0 + r) * 16 + wave * kBlocksPerWave + t,
                                        a.table_stride - 1)]
                            : 0;
    const unsigned probe = gate.probe();

    count = position + 1;
    const int nsplit = (count + kSplitKeys - 1) / kSplitKeys;
    // A context the grid or the block table cannot cover is an error, never
    // a partial read: flag it once, and the unit computes nothing.
    const bool covered =
        count >= 1 && nsplit <= a.max_splits && count <= a.table_stride * kBlockPos;
    if (exists && !covered && split0 == 0 && wave == 0 && lane == 0) atomicOr(a.status, 2);
    const bool live = covered && split0 * kSplitKeys < count;  // uniform per unit
    // Blocks of this wave that hold keys load; the others load nothing
    // (their keys are masked below). With `early`, the K of every block but
    // the context's last is requested before the gate: a unit that waits for
    // its inputs has it in flight meanwhile. Their V, the last block (it holds
    // the key this step appends) and q come after.
    const int stream_blocks = (count + kBlockPos - 1) / kBlockPos;
    const float *layer_kv = a.kv + (size_t)a.layer * a.layer_stride;
    bool bad_block = false;
    float4 kr[kBlocksPerWave][4], vr[kBlocksPerWave][4];
    // sel 0: blocks before the context's last (zeros past the context);
    // 1: the context's last block only; 2: every block.
    auto load = [&](int r, bool values, int sel) {
#pragma unroll
        for (int t = 0; t < kBlocksPerWave; t++) {
            float4 *dst = values ? vr[t] : kr[t];
            const int b = (split0 + r) * 16 + wave * kBlocksPerWave + t;
            const bool in = b < stream_blocks, last = b == stream_blocks - 1;  // uniform
            if (in && (sel == 2 || (sel == 1) == last)) {
                // An id outside the pool is flagged and replaced.
                bad_block |= (unsigned)ids[r][t] >= a.blocks;
                const int id = (unsigned)ids[r][t] < a.blocks ? ids[r][t] : 0;
                const float *tile = layer_kv + ((size_t)id * kHeads + head) * 2048 +
                                    (values ? 1024 : 0) + lane * 4;
#pragma unroll
                for (int i = 0; i < 4; i++) dst[i] = stream_load(tile + i * 256);
            } else if (!in && sel != 1) {
#pragma unroll
                for (int i = 0; i < 4; i++) dst[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    constexpr bool TQ = GateTaggedQkv<Gate>::value;
    if (live && (early || TQ)) load(0, false, TQ ? 2 : 0);
    if (live && TQ) load(0, true, 2);
    gate.pass(probe, live);
    // V after the gate: it is needed after the scores, and requesting it
    // before the gate only deepens the memory queues every other task waits
    // in (measured on MI355X at B=64: 696 vs 701 us per step).
    if (live && early && !TQ) load(0, true, 0);

    if (live) {
        float4 q, knew = {}, vnew = {};
        // The appended key (index count - 1): its block, and its slot there
        // (float4 kk / 4 of the lanes of key row kk % 4).
        const int cur_block = (count - 1) >> 4, kk = (count - 1) & 15;
        auto patch = [&](int r, float4(&regs)[kBlocksPerWave][4], const float4 &v) {
#pragma unroll
            for (int t = 0; t < kBlocksPerWave; t++)
                if ((split0 + r) * 16 + wave * kBlocksPerWave + t == cur_block &&
                    krow == (kk & 3)) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (i == (kk >> 2)) regs[t][i] = v;
                }
        };
        if constexpr (TQ) {
            gate.poll_qkv(s, head, dcol, q, knew, vnew);
            patch(0, kr, knew);
            patch(0, vr, vnew);
        } else {
            load(0, false, early ? 1 : 2);
            load(0, true, early ? 1 : 2);
            q = *(const float4 *)(a.q + (size_t)s * kWidth + head * kHeadDim + dcol * 4);
        }
#pragma unroll
        for (int r = 0; r < ROUNDS; r++) {
            if (r >= rounds || (split0 + r) * kSplitKeys >= count) break;  // uniform
            const bool next = r + 1 < rounds && (split0 + r + 1) * kSplitKeys < count;
            const int first_block = (split0 + r) * 16 + wave * kBlocksPerWave;
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
            if (next) {
                load(r + 1, false, 2);
                if constexpr (TQ) patch(r + 1, kr, knew);
            }
            m = xor16_32_max(m);
#pragma unroll
            for (int t = 0; t < kBlocksPerWave; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // Slots past the context hold whatever the pool held
                    // before: they are skipped, never multiplied by a zero
                    // weight.
                    if (score[t][i] == -INFINITY) continue;
                    const float e = expf(score[t][i] - m);
                    l += e;
                    acc.x = fmaf(e, vr[t][i].x, acc.x);
                    acc.y = fmaf(e, vr[t][i].y, acc.y);
                    acc.z = fmaf(e, vr[t][i].z, acc.z);
                    acc.w = fmaf(e, vr[t][i].w, acc.w);
                }
            if (next) {
                load(r + 1, true, 2);
                if constexpr (TQ) patch(r + 1, vr, vnew);
            }
            // Lanes of one key row hold the same l; sum the four rows.
            l = xor16_32_sum(l);
            acc.x = xor16_32_sum(acc.x);
            acc.y = xor16_32_sum(acc.y);
            acc.z = xor16_32_sum(acc.z);
            acc.w = xor16_32_sum(acc.w);
            if (lane < 16) sh[r].acc[wave][lane] = acc;
            if (lane == 0) {
                sh[r].m[wave] = m;
                sh[r].l[wave] = l;
            }
        }
        if (bad_block && lane == 0) atomicOr(a.status, 2);
    }
    __syncthreads();
    const int state = live ? UNIT_LIVE : (exists && !covered ? UNIT_UNCOVERED : UNIT_EMPTY);
    if (!live || wave >= merge_waves || lane >= 16) return state;

    // Merge the unit's waves (fixed order), per split. A wave without keys
    // has l = 0.
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        if (r >= rounds || (split0 + r) * kSplitKeys >= count) break;
        float m = sh[r].m[0];
#pragma unroll
        for (int w = 1; w < kUnitWaves; w++) m = fmaxf(m, sh[r].m[w]);
        float l = 0.0f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < kUnitWaves; w++) {
            if (sh[r].l[w] == 0.0f) continue;
            const float f = expf(sh[r].m[w] - m);
            l = fmaf(sh[r].l[w], f, l);
            const float4 x = sh[r].acc[w][lane];
            acc.x = fmaf(x.x, f, acc.x);
            acc.y = fmaf(x.y, f, acc.y);
            acc.z = fmaf(x.z, f, acc.z);
            acc.w = fmaf(x.w, f, acc.w);
        }
        mm[r] = m;
        ll[r] = l;
        aa[r] = acc;
    }
    return state;
}

// attend_unit, then the split's (max, sum, unnormalised P.V) partial into
// the pgpu_attention_scratch layout.
__device__ inline void attend_split(const AttnArgs &a, int head, int split, int s, int wave,
                                    AttnShared &sh, bool exists = true) {
    float4 aa;
    float mm, ll;
    int count;
    const int state = attend_unit(a, head, split, s, wave, &sh, exists, &aa, &mm, &ll, count);
    const int lane = threadIdx.x & 63;
    if (state != UNIT_LIVE || wave != 0 || lane >= 16) return;
    const size_t slot = ((size_t)s * kHeads + head) * a.max_splits + split;
    *(float4 *)(a.part_acc + slot * 64 + lane * 4) = aa;
    if (lane == 0) *(float2 *)(a.part_ml + slot * 2) = make_float2(mm, ll);
}

}  // namespace pgpu
