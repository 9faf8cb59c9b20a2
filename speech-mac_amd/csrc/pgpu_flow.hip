// One-launch decode step: every layer of a batched decode step
// (phonon_flow_stack_step, src/phonon_transformer.c:455-482, for B streams)
// in a single kernel launch, as a dataflow graph of work-group tasks.
//
// Why: a step is 5 dependent phases per layer. Run as one launch per phase,
// every phase boundary drains and refills the whole GPU, and the
// latency-bound projections (~1-3 MB of weights) serialise with the
// HBM-bound attention (~270 MB of K/V per layer at B=64). Here the phases
// are per 16-stream tile: tile t's projection chain (out, MLP, next QKV)
// runs while other tiles' attention streams K/V, and no launch gap separates
// the phases.
//
// Scheduling. Work-group i runs the task of schedule[i] (pgpu_flow_task).
// The host lists the tasks so that every task comes after the tasks it
// depends on. Work-groups are dispatched in index order, so the
// lowest-numbered unfinished task always has its inputs done and is running
// or about to be dispatched: the launch cannot deadlock. A task that
// starts before its inputs are ready waits (one lane polls a counter) while
// holding its slot.
//
// Synchronisation without cache maintenance. Each XCD has its own L2, and
// an agent-scope fence writes back or invalidates a whole L2. Instead
// (counter mode, f.tagged = 0):
//  - every value a task writes for another task is stored write-through at
//    device scope (global_store ... sc1: pgpu_gemm.hpp store_wt), and the
//    storing waves drain vmcnt before the task's counter is incremented;
//  - every such value lives at an address that no task reads before it is
//    written within the launch (activations, partials and merged outputs
//    have one buffer per layer; an appended K/V slot is read only by the
//    attention of its own layer), so a consumer's plain load cannot hit a
//    stale line in its L1 or L2: caches start the launch clean;
//  - counters are atomics; a waiting lane polls with device-scope loads.
// Read-only operands (weights, norms, positions, block tables, the RoPE
// table, older K/V) are plain loads and stay cacheable.
//
// Tagged mode (f.tagged = PGPU_FLOW_HANDOFF_TAGGED, for a batch of a few
// streams): the layer output x, the out projection r, the merged attention
// rows and the split partials are tagged words (pgpu_gemm.hpp TagPoll),
// stored without a drain; the consumer polls the words themselves, so a
// hand-off costs one memory round trip less. A consumer first waits (one
// lane, one counter) for the phase before its producers, so that tasks
// dispatched long before their inputs do not poll all that time. Polls
// fetch from memory on every round (device scope), which with many streams
// per tile costs more than the counter mode's shared, cacheable loads
// (measured), hence the modes. q, the appended K/V and the MLP hidden
// fragments keep their counters in all of them.
//
// Tagged partials (f.tagged = PGPU_FLOW_HANDOFF_PARTS): only the split
// partials are tagged. An attention task that does not complete its
// (stream, head) then ends right after its split count, without waiting for
// its partial stores to reach memory (the drain took about a quarter of an
// attention task's life at 64 streams); the task that completes the group
// polls the 66 words of each partial, which is cheap, and hands the merged
// row over as in the counter mode.
//
// Every wait is bounded (1 s of the 100 MHz constant clock): a task that
// times out sets status bit 4, and every other waiter then stops waiting,
// so the launch always ends.
#include "pgpu_attention.hpp"
#include "pgpu_gemm.hpp"
#include "phonon_gpu.h"

namespace pgpu {
namespace {

constexpr uint64_t kWaitTicks = 100000000ull;  // 1 s at 100 MHz

__device__ inline unsigned *phase_counter(const pgpu_flow_step &f, int layer, int tile,
                                          int kind) {
    return f.phase + ((size_t)(layer * f.tiles + tile) * PGPU_FLOW_KINDS + kind) *
                         PGPU_FLOW_COUNTER_STRIDE;
}

// Wait until a counter holds at least `target` (no wait if `flag` is null):
// one lane polls, then the work-group barrier releases the rest. probe()
// issues the first check on its own, so that a task can send it together
// with its other first loads and pass() only polls again if that check
// found the count short.
struct FlowWait {
    const unsigned *flag;
    unsigned target;
    int *status;
    uint64_t ticks;  // give-up bound on the 100 MHz constant clock
    __device__ unsigned probe() const {
        return threadIdx.x == 0 && flag
                   ? __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : target;
    }
    // `first` is probe()'s value; needed = false skips the wait (the task
    // found it has nothing to do). Every thread must call it.
    __device__ void pass(unsigned first, bool needed = true) const {
        if (threadIdx.x == 0 && needed && first < target) {
            const uint64_t t0 = wall_clock64();
            // The counter and the status word are loaded together: one
            // round trip to memory per poll.
            for (;;) {
                const unsigned count =
                    __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int st = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (count >= target) break;
                if ((st & 4) || wall_clock64() - t0 > ticks) {
                    atomicOr(status, 4);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        __syncthreads();
    }
    __device__ void operator()() const { pass(probe()); }
};

// Waits give up after f.wait_us microseconds (0: 1 s).
__device__ inline uint64_t wait_ticks(const pgpu_flow_step &f) {
    return f.wait_us ? (uint64_t)f.wait_us * 100u : kWaitTicks;
}

__device__ inline FlowWait wait_for(const pgpu_flow_step &f, int layer, int tile, int kind,
                                    unsigned target) {
    return FlowWait{phase_counter(f, layer, tile, kind), target, f.status, wait_ticks(f)};
}

// Task timeline (optional): slot 0 = start, 1 = inputs ready, 2 = end,
// 3 = where it ran: XCC id << 32 | HW_ID (CU, shader array and engine).
__device__ inline void trace_mark(const pgpu_flow_step &f, int slot) {
    if (!f.trace || threadIdx.x != 0) return;
    f.trace[(size_t)blockIdx.x * 4 + slot] = wall_clock64();
    if (slot == 0) {
        const uint32_t xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);  // HW_REG_XCC_ID[3:0]
        const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_REG_HW_ID
        f.trace[(size_t)blockIdx.x * 4 + 3] = (uint64_t)xcc << 32 | hw;
    }
}

// Completes a task: every wave's write-through stores have drained, then
// one lane counts the task (and, if given, a second counter).
__device__ inline void flow_signal(const pgpu_flow_step &f, unsigned *flag,
                                   unsigned *also = nullptr) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (also) __hip_atomic_fetch_add(also, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    trace_mark(f, 2);
}

// FlowWait that also records when the inputs were ready.
struct TracedWait {
    FlowWait w;
    const pgpu_flow_step *f;
    __device__ unsigned probe() const { return w.probe(); }
    __device__ void pass(unsigned first, bool needed = true) const {
        w.pass(first, needed);
        trace_mark(*f, 1);
    }
    __device__ void operator()() const { pass(probe()); }
};

// Per-layer activation rows [tiles*16][512]: 0 = layer output x, 1 = r (out
// projection + residual), 2 = q, 3 = merged attention output.
__device__ inline float *act_rows(const pgpu_flow_step &f, int layer, int which) {
    return f.act + ((size_t)layer * 4 + which) * (size_t)f.tiles * 16 * kWidth;
}

__device__ inline float *layer_output(const pgpu_flow_step &f, int layer) {
    return layer + 1 == f.layer_count ? f.output : act_rows(f, layer, 0);
}

__device__ inline const float *layer_input(const pgpu_flow_step &f, int layer) {
    return layer == 0 ? f.input : act_rows(f, layer - 1, 0);
}

__device__ inline uint16_t *hidden_rows(const pgpu_flow_step &f, int layer) {
    return f.hidden + (size_t)layer * f.tiles * (kFfn / 32) * 1536;
}

// Tagged mode: per-layer rows [tiles*16][512] of tagged words: 0 = layer
// output x, 1 = r, 2 = merged attention output.
// Merge-in-out mode adds 3 = q (scaled), 4 = k, 5 = v of the QKV tasks.
enum { ROWS_X = 0, ROWS_R = 1, ROWS_ATTN = 2, ROWS_Q = 3, ROWS_KINDS = 6 };
__device__ inline uint64_t *tagged_rows(const pgpu_flow_step &f, int layer, int which) {
    return f.rows + ((size_t)layer * ROWS_KINDS + which) * (size_t)f.tiles * 16 * kWidth;
}

// Fused MLP: MLP_IN task `task`'s partial of `layer`, [16 streams][512]
// fp32.
__device__ inline float *fused_parts(const pgpu_flow_step &f, int layer, int task) {
    return f.mlp_parts + ((size_t)layer * PGPU_FLOW_MLP_IN_TASKS + task) * 16 * kWidth;
}

// Fused MLP, after the last layer: output dimensions [64 index, 64 index +
// 64) of each stream (wave n: stream n of the tile) = r + the layer's MLP
// partials, summed as the QKV prologue sums them (fused_sum), stored plainly
// (read after the launch).
__device__ inline void fused_output_task(const pgpu_flow_step &f, int layer, int tile, int index,
                                         uint32_t tag) {
    wait_for(f, layer, tile, PGPU_FLOW_MLP_IN, PGPU_FLOW_MLP_IN_TASKS)();
    trace_mark(f, 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int d = index * kHeadDim + (threadIdx.x & 63);
    bool bad = false;
    if (wave < min(PGPU_FLOW_FUSED_MAX_STREAMS, f.streams - tile * 16)) {  // uniform
        const int s = tile * 16 + wave;
        const float x = fused_sum(tagged_rows(f, layer, ROWS_R) + (size_t)s * kWidth,
                                  fused_parts(f, layer, 0), 16, s, d,
                                  TagPoll{tag, f.status, wait_ticks(f), false});
        f.output[(size_t)s * kWidth + d] = x;
        bad = !isfinite(x);
    }
    flag_nonfinite(f.status, bad);
    trace_mark(f, 2);
}

// Attention gate of the merge-in-out mode (outside a prefill): a first wait
// for one of the head's QKV tasks (a count without a drain), then the
// unit's q and the appended key's K and V polled as tagged words
// (attend_unit: GateTaggedQkv).
struct TaggedQkvGate {
    static constexpr bool kTaggedQkv = true;
    FlowWait hint;
    const uint64_t *qkv;  // the layer's tagged q rows; k and v follow, `part` words apart
    size_t part;
    TagPoll tp;
    const pgpu_flow_step *f;  // for the task trace's inputs-ready mark
    __device__ unsigned probe() const { return hint.probe(); }
    __device__ void pass(unsigned first, bool needed) const { hint.pass(first, needed); }
    // Dimensions [4 dcol, 4 dcol + 4) of head `head` of stream s.
    __device__ void poll_qkv(int s, int head, int dcol, float4 &q, float4 &k, float4 &v) const {
        const __amdgpu_buffer_rsrc_t r = tag_rsrc(qkv, (uint32_t)(3 * part * 8));
        const uint32_t off = (uint32_t)(((size_t)s * kWidth + head * kHeadDim + dcol * 4) * 8);
        const uint32_t step = (uint32_t)(part * 8);
        u32x4 w[6];
        const uint64_t t0 = wall_clock64();
        for (int round = 0;; round++) {
            __asm__ volatile("" ::: "memory");
            bool ok = true;
#pragma unroll
            for (int p = 0; p < 3; p++) {
                w[2 * p] = tag_load2(r, off + p * step);
                w[2 * p + 1] = tag_load2(r, off + p * step + 16);
                ok &= tag_ok2(w[2 * p], tp.tag) && tag_ok2(w[2 * p + 1], tp.tag);
            }
            if (__all(ok)) break;
            if (tag_give_up(tp, t0, round)) break;
            __builtin_amdgcn_s_sleep(1);
        }
        q = make_float4(bitsf(w[0].x), bitsf(w[0].z), bitsf(w[1].x), bitsf(w[1].z));
        k = make_float4(bitsf(w[2].x), bitsf(w[2].z), bitsf(w[3].x), bitsf(w[3].z));
        v = make_float4(bitsf(w[4].x), bitsf(w[4].z), bitsf(w[5].x), bitsf(w[5].z));
        trace_mark(*f, 1);
    }
};

__device__ inline GemmArgs base_args(const pgpu_flow_step &f, const pgpu_flow_layer &ly,
                                     int which, uint32_t tag) {
    GemmArgs a{};
    a.w = ly.values[which];
    a.wscale = ly.scales[which];
    a.streams = f.streams;
    a.status = f.status;
    a.wt_out = true;  // read by tasks on other XCDs within the launch
    a.tp = TagPoll{tag, f.status, wait_ticks(f), false};
    a.pos_delta = f.pos_delta;
    return a;
}

// Tagged mode: the wait before a task polls its tagged inputs (the count of
// the phase before its producers, or none).
__device__ inline FlowWait no_wait(const pgpu_flow_step &f) {
    return FlowWait{nullptr, 0u, f.status, 0u};
}

// ATTN task: splits [unit, unit + 1) x f.attn_rounds of (stream t*16 + n,
// head), one after the other. Each split's partial goes
// to its slot of the (layer, stream, head) group; the task whose splits
// complete the group's count (nsplit) merges all partials in split order
// into the attention row, with the arithmetic of the single-phase merge. A
// task that holds every split merges them from registers. A task past the
// context ends without a trace; if the context is not covered, pair 0
// completes the (stream, head) with a zero row (the unit flags it).
constexpr int kFlowRounds = PGPU_FLOW_ATTN_ROUNDS;
static_assert(kFlowRounds * sizeof(AttnShared) <= kTaskLds * 2, "attention LDS");

// Tagged partials, after the unit. Wave 1 stores every split's partial as
// a tagged record and ends; wave 0 counts the splits (it does not wait for
// wave 1's stores: each wave's memory operations retire in order, and only
// its own), and if its count completes the group it polls all records and
// merges them in split order (the arithmetic of the counter mode). A task
// that holds every split merges from registers. With `rows_tagged` the
// merged row goes out as tagged words, then the tile's ATTN count (a hint
// for the MLP-in tasks' first wait); otherwise it is stored write-through
// and drained before the count, as in the counter mode.
template <int R>
__device__ inline void tagged_attention_tail(const pgpu_flow_step &f, int layer, int tile, int s,
                                             int head, int split0, int nsplit, int rounds,
                                             bool covered, const float4 *aa, const float *mm,
                                             const float *ll, size_t group, uint32_t tag,
                                             bool rows_tagged, int wave) {
    const int lane = threadIdx.x & 63, d = (lane & 15) * 4;
    uint64_t *part = f.parts + group * f.max_splits * PGPU_FLOW_PART_WORDS;
    const bool in_registers = covered && nsplit <= R;
    if (wave == 1) {
        if (covered && !in_registers) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                if (r >= rounds) break;
                uint64_t *rec = part + (size_t)(split0 + r) * PGPU_FLOW_PART_WORDS;
                if (lane < 16) store_tagged4(rec + d, aa[r], tag);
                if (lane == 0) {
                    store_tagged(rec + 64, mm[r], tag);
                    store_tagged(rec + 65, ll[r], tag);
                }
            }
        }
        return;
    }
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    bool bad = false;
    if (in_registers) {
        float mx = -INFINITY, total = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r >= nsplit) break;
            const float acc[4] = {aa[r].x, aa[r].y, aa[r].z, aa[r].w};
            merge_step(mx, total, v, 4, mm[r], ll[r], acc);
        }
        bad = merge_finish<4>(total, v);
    } else if (covered) {
        unsigned done = 0;
        if (lane == 0)
            done = __hip_atomic_fetch_add(f.split_done + group, (unsigned)rounds,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        done = __shfl(done, 0);
        if (done + rounds != (unsigned)nsplit) {
            trace_mark(f, 2);
            return;
        }
        float mx = -INFINITY, total = 0.0f;
        merge_tagged_splits(part, 0, nsplit, mx, total, v,
                            TagPoll{tag, f.status, wait_ticks(f), false});
        bad = merge_finish<4>(total, v);
    }
    if (!rows_tagged) {
        if (lane < 16)
            store_wt(act_rows(f, layer, 3) + (size_t)s * kWidth + head * kHeadDim + d,
                     make_float4(v[0], v[1], v[2], v[3]));
        flag_nonfinite(f.status, bad && lane < 16);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        if (lane < 16)
            store_tagged4(tagged_rows(f, layer, ROWS_ATTN) + (size_t)s * kWidth +
                              head * kHeadDim + d,
                          make_float4(v[0], v[1], v[2], v[3]), tag);
        flag_nonfinite(f.status, bad && lane < 16);
    }
    if (lane == 0)
        __hip_atomic_fetch_add(phase_counter(f, layer, tile, PGPU_FLOW_ATTN), 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    trace_mark(f, 2);
}

template <int MODE, bool PRE, int R>
__device__ inline void attention_task(const pgpu_flow_step &f, const pgpu_paged_kv &kv,
                                      int layer, int tile, int index, AttnShared *sh,
                                      uint32_t tag) {
    const int head = index & 7, split0 = ((index >> 3) & 255) * R, n = index >> 11;
    const int s = tile * 16 + n;
    if (s >= f.streams) return;  // uniform
    const TracedWait ready{
        PRE
            ? wait_for(f, layer, 0, PGPU_FLOW_QKV_ALL, (unsigned)(PGPU_FLOW_QKV_TASKS * f.tiles))
            : wait_for(f, layer, tile, PGPU_FLOW_QKV_HEAD + head, 3u),
        &f};

    AttnArgs a;
    a.q = act_rows(f, layer, 2);
    a.kv = kv.base;
    a.layer_stride = kv.layer_stride;
    a.blocks = (unsigned)kv.blocks;
    a.layer = layer + f.pool_offset;
    a.tables = f.tables;
    a.table_stride = f.table_stride;
    a.positions = f.positions;
    a.pos_delta = f.pos_delta;
    a.streams = f.streams;
    a.max_splits = f.max_splits;
    a.part_acc = nullptr;
    a.part_ml = nullptr;
    a.status = f.status;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float4 aa[R];
    float mm[R], ll[R];
    int count;
    constexpr bool tagged_parts = MODE != PGPU_FLOW_HANDOFF_COUNTER;
    constexpr bool MO =
        MODE == PGPU_FLOW_HANDOFF_MERGE_OUT || MODE == PGPU_FLOW_HANDOFF_FUSED_MLP;
    int state;
    if constexpr (MO && !PRE) {
        const TaggedQkvGate gate{wait_for(f, layer, tile, PGPU_FLOW_QKV_HEAD + head, 1u),
                                 tagged_rows(f, layer, ROWS_Q),
                                 (size_t)f.tiles * 16 * kWidth,
                                 TagPoll{tag, f.status, wait_ticks(f), false}, &f};
        state = attend_unit<R>(a, head, split0, s, wave, sh, true, aa, mm, ll, count, gate, R,
                               true, 1);
    } else {
        state = attend_unit<R>(a, head, split0, s, wave, sh, true, aa, mm, ll, count, ready, R,
                               !PRE, tagged_parts && !MO ? 2 : 1);
    }
    if constexpr (MO) {
        // Every split's partial goes out as a tagged record; the tile's
        // out-projection tasks poll and merge them.
        if (wave != 0 || state != UNIT_LIVE) return;
        const int lane = threadIdx.x & 63;
        const size_t group = ((size_t)layer * f.tiles * 16 + s) * kHeads + head;
        uint64_t *part = f.parts + group * f.max_splits * PGPU_FLOW_PART_WORDS;
        const int nsplit = (count + kSplitKeys - 1) / kSplitKeys;
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r >= R || split0 + r >= nsplit) break;
            uint64_t *rec = part + (size_t)(split0 + r) * PGPU_FLOW_PART_WORDS;
            if (lane < 16) store_tagged4(rec + lane * 4, aa[r], tag);
            if (lane == 0) {
                store_tagged(rec + 64, mm[r], tag);
                store_tagged(rec + 65, ll[r], tag);
            }
        }
        trace_mark(f, 2);
        return;
    }
    if (wave > (tagged_parts ? 1 : 0) || state == UNIT_EMPTY ||
        (state == UNIT_UNCOVERED && split0 != 0))
        return;
    const bool covered = state == UNIT_LIVE;
    const int nsplit = (count + kSplitKeys - 1) / kSplitKeys;
    const int rounds = min(R, nsplit - split0);  // splits of this task (if covered)

    const int lane = threadIdx.x & 63, d = (lane & 15) * 4;
    const size_t group = ((size_t)layer * f.tiles * 16 + s) * kHeads + head;
    if constexpr (tagged_parts) {
        tagged_attention_tail<R>(f, layer, tile, s, head, split0, nsplit, rounds, covered, aa, mm,
                              ll, group, tag, MODE == PGPU_FLOW_HANDOFF_TAGGED, wave);
        return;
    }
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    bool finish = !covered, bad = false;
    if (covered && nsplit <= R) {
        float mx = -INFINITY, total = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r >= nsplit) break;
            const float acc[4] = {aa[r].x, aa[r].y, aa[r].z, aa[r].w};
            merge_step(mx, total, v, 4, mm[r], ll[r], acc);
        }
        bad = merge_finish<4>(total, v);
        finish = true;
    } else if (covered) {
        float *acc = f.part_acc + group * f.max_splits * 64;
        float *ml = f.part_ml + group * f.ml_group;
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r >= rounds) break;
            if (lane < 16) store_wt(acc + (split0 + r) * 64 + d, aa[r]);
            if (lane == 0) store_wt((float2 *)(ml + 2 * (split0 + r)), make_float2(mm[r], ll[r]));
        }
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned done = 0;
        if (lane == 0)
            done = __hip_atomic_fetch_add(f.split_done + group, (unsigned)rounds,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        done = __shfl(done, 0);
        if (done + rounds == (unsigned)nsplit) {
            bad = merge_splits<4>(acc, ml, nsplit, d, v);
            finish = true;
        }
    }
    if (!finish) {
        trace_mark(f, 2);
        return;
    }
    if (lane < 16)
        store_wt(act_rows(f, layer, 3) + (size_t)s * kWidth + head * kHeadDim + d,
                 make_float4(v[0], v[1], v[2], v[3]));
    flag_nonfinite(f.status, bad && lane < 16);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0)
        __hip_atomic_fetch_add(phase_counter(f, layer, tile, PGPU_FLOW_ATTN), 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    trace_mark(f, 2);
}

// MODE: the launch's hand-off mode (PGPU_FLOW_HANDOFF_*, f.tagged), one
// kernel per mode, so that no mode's code carries another's registers.
template <bool Q8, int MODE, bool PRE, int R>
__device__ inline void flow_step_task(const pgpu_flow_step &f, const pgpu_paged_kv &kv,
                                      uint4 *lds4) {
    uint16_t *lds = (uint16_t *)lds4;
    trace_mark(f, 0);
    const uint32_t desc = f.schedule[blockIdx.x];
    // The next step's counters: zeroed by the first work-groups, one 16-byte
    // store per lane (no task of this step reads them; the launch boundary
    // orders the stores before the next step).
    if (blockIdx.x * PGPU_FLOW_CLEAR_WORDS < f.clear_words) {
        const unsigned i = blockIdx.x * PGPU_FLOW_CLEAR_WORDS + threadIdx.x * 4;
        if (i < f.clear_words) *(uint4 *)(f.clear + i) = make_uint4(0u, 0u, 0u, 0u);
    }
    const uint32_t tag = MODE != PGPU_FLOW_HANDOFF_COUNTER ? f.tag : 0u;
    const int kind = desc & 7, layer = (desc >> 3) & 63, tile = (desc >> 9) & 255,
              index = desc >> 17;
    const pgpu_flow_layer &ly = f.layers[layer];
    const float *norm = ly.norms;
    const int live = min(16, f.streams - tile * 16);
    constexpr bool fused = MODE == PGPU_FLOW_HANDOFF_FUSED_MLP && !PRE;
    constexpr bool merge_out = MODE == PGPU_FLOW_HANDOFF_MERGE_OUT || fused;
    constexpr bool tagged = merge_out || MODE == PGPU_FLOW_HANDOFF_TAGGED;
    const bool last = layer + 1 == f.layer_count;
    uint64_t *const ready_mark =
        tagged && f.trace ? f.trace + (size_t)blockIdx.x * 4 + 1 : nullptr;
    switch (kind) {
    case PGPU_FLOW_QKV: {
        GemmArgs a = base_args(f, ly, 0, tag);
        a.ln_w = norm;
        a.ln_b = norm + kWidth;
        a.ln_eps = 1e-5f;
        a.n_rows = 3 * kWidth;
        a.k_cols = kWidth;
        a.q_out = act_rows(f, layer, 2);
        a.kv = kv.base;
        a.layer_stride = kv.layer_stride;
        a.blocks = (unsigned)kv.blocks;
        a.layer = layer + f.pool_offset;
        a.tables = f.tables;
        a.table_stride = f.table_stride;
        a.positions = f.positions;
        a.rope = (const float2 *)f.rope;
        if constexpr (tagged) {
            // The previous layer's output, polled once its MLP-in tasks are
            // done (the phase before its producers; with the fused MLP, the
            // MLP-in tasks are its producers, and their count is the wait).
            a.ln_x = layer == 0 ? f.input : nullptr;
            a.tx = layer == 0 ? nullptr : tagged_rows(f, layer - 1, ROWS_X);
            a.ready_mark = ready_mark;
            if constexpr (merge_out && !PRE) {
                // q, k and v also go out as tagged words for the attention
                // units; the pool's K/V are read by later launches only.
                a.tqkv = tagged_rows(f, layer, ROWS_Q);
                a.tqkv_part = (size_t)f.tiles * 16 * kWidth;
            }
            const FlowWait w = layer == 0 ? no_wait(f)
                                          : wait_for(f, layer - 1, tile, PGPU_FLOW_MLP_IN,
                                                     PGPU_FLOW_MLP_IN_TASKS);
            bool done = false;
            if constexpr (fused) {
                if (layer > 0) {
                    // x = r + the previous layer's MLP partials; tasks 0..7
                    // hand 64 dimensions each on to the out projection.
                    a.tx = nullptr;
                    a.tres = tagged_rows(f, layer - 1, ROWS_R);
                    a.tmlp = fused_parts(f, layer - 1, 0);
                    a.mlp_streams = 16;
                    a.tpub = tagged_rows(f, layer - 1, ROWS_X);
                    a.pub0 = index < kHeads ? index * kHeadDim : -1;
                    gemm_wide_task<SRC_LN_PARTS, EPI_QKV, Q8>(a, index, tile, lds, w);
                    done = true;
                }
            }
            if (!done) gemm_wide_task<SRC_LN, EPI_QKV, Q8>(a, index, tile, lds, w);
            if constexpr (merge_out && !PRE) {
                // A count for first waits only: no drain.
                __syncthreads();
                if (threadIdx.x == 0)
                    __hip_atomic_fetch_add(
                        phase_counter(f, layer, tile, PGPU_FLOW_QKV_HEAD + (index & 7)), 1u,
                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                trace_mark(f, 2);
                break;
            }
        } else {
            a.ln_x = layer_input(f, layer);
            const FlowWait w = layer == 0 ? no_wait(f)
                                          : wait_for(f, layer - 1, tile, PGPU_FLOW_MLP_OUT,
                                                     PGPU_FLOW_MLP_OUT_TASKS);
            gemm_wide_task<SRC_LN, EPI_QKV, Q8>(a, index, tile, lds, TracedWait{w, &f});
        }
        // Rows [64 index, +64): q, k or v of head index % 8.
        flow_signal(f, phase_counter(f, layer, tile, PGPU_FLOW_QKV_HEAD + (index & 7)),
                    PRE ? phase_counter(f, layer, 0, PGPU_FLOW_QKV_ALL) : nullptr);
        break;
    }
    case PGPU_FLOW_ATTN:
        attention_task<MODE, PRE, R>(f, kv, layer, tile, index, (AttnShared *)lds4, tag);
        break;
    case PGPU_FLOW_OUT: {
        GemmArgs a = base_args(f, ly, 1, tag);
        a.n_rows = kWidth;
        a.k_cols = kWidth;
        a.ld_out = kWidth;
        if constexpr (tagged) {
            // Merged attention rows, polled once the tile's QKV tasks are
            // done (head 7's are listed last).
            a.tx = tagged_rows(f, layer, ROWS_ATTN);
            a.tout = tagged_rows(f, layer, ROWS_R);
            a.residual = layer == 0 ? f.input : nullptr;
            a.tres = layer == 0 ? nullptr : tagged_rows(f, layer - 1, ROWS_X);
            a.ready_mark = ready_mark;
            const FlowWait w =
                PRE ? wait_for(f, layer, 0, PGPU_FLOW_QKV_ALL,
                                     (unsigned)(PGPU_FLOW_QKV_TASKS * f.tiles))
                          : wait_for(f, layer, tile, PGPU_FLOW_QKV_HEAD + kHeads - 1, 3u);
            if constexpr (merge_out) {
                // The split partials of the tile's streams, merged here.
                a.tparts = f.parts + (size_t)layer * f.tiles * 16 * kHeads * f.max_splits *
                                         PGPU_FLOW_PART_WORDS;
                a.positions = f.positions;
                a.max_splits = f.max_splits;
                a.table_stride = f.table_stride;
                gemm_wide_task<SRC_ATTN_TAGGED, EPI_RESIDUAL, Q8>(a, index, tile, lds, w);
            } else {
                gemm_wide_task<SRC_ROWS, EPI_RESIDUAL, Q8>(a, index, tile, lds, w);
            }
            trace_mark(f, 2);
        } else {
            a.ln_x = act_rows(f, layer, 3);
            a.out = act_rows(f, layer, 1);
            a.residual = layer_input(f, layer);
            gemm_wide_task<SRC_ROWS, EPI_RESIDUAL, Q8>(
                a, index, tile, lds,
                TracedWait{wait_for(f, layer, tile, PGPU_FLOW_ATTN, (unsigned)(kHeads * live)),
                           &f});
            flow_signal(f, phase_counter(f, layer, tile, PGPU_FLOW_OUT));
        }
        break;
    }
    case PGPU_FLOW_MLP_IN: {
        GemmArgs a = base_args(f, ly, 2, tag);
        a.ln_w = norm + 2 * kWidth;
        a.ln_b = norm + 3 * kWidth;
        a.ln_eps = 1e-5f;
        a.n_rows = kFfn;
        a.k_cols = kWidth;
        a.out_split = hidden_rows(f, layer);
        a.out_kb = kFfn / 32;
        if constexpr (fused) {
            // r polled as in MERGE_OUT; the task's partial of the MLP-out
            // projection is stored write-through, drained and counted
            // (flow_signal below).
            a.tx = tagged_rows(f, layer, ROWS_R);
            a.ready_mark = ready_mark;
            a.w2 = ly.values[3];
            a.w2scale = ly.scales[3];
            a.tmlp_out = fused_parts(f, layer, index);
            gemm_wide_task<SRC_LN, EPI_GELU_W2, Q8>(
                a, index, tile, lds, wait_for(f, layer, tile, PGPU_FLOW_QKV_HEAD + kHeads - 1, 3u));
        } else if constexpr (tagged) {
            // r, polled once every (stream, head) of the tile is merged
            // (with the merge in the out projection: once the tile's QKV
            // tasks are done, as the out projection itself).
            a.tx = tagged_rows(f, layer, ROWS_R);
            a.ready_mark = ready_mark;
            gemm_wide_task<SRC_LN, EPI_GELU_SPLIT, Q8>(
                a, index, tile, lds,
                merge_out ? wait_for(f, layer, tile, PGPU_FLOW_QKV_HEAD + kHeads - 1, 3u)
                          : wait_for(f, layer, tile, PGPU_FLOW_ATTN, (unsigned)(kHeads * live)));
        } else {
            a.ln_x = act_rows(f, layer, 1);
            gemm_wide_task<SRC_LN, EPI_GELU_SPLIT, Q8>(
                a, index, tile, lds,
                TracedWait{wait_for(f, layer, tile, PGPU_FLOW_OUT, PGPU_FLOW_OUT_TASKS), &f});
        }
        flow_signal(f, phase_counter(f, layer, tile, PGPU_FLOW_MLP_IN));
        break;
    }
    case PGPU_FLOW_MLP_OUT: {
        if constexpr (fused) {
            fused_output_task(f, layer, tile, index, tag);
            break;
        }
        GemmArgs a = base_args(f, ly, 3, tag);
        a.xs = hidden_rows(f, layer);
        a.n_rows = kWidth;
        a.k_cols = kFfn;
        a.ld_out = kWidth;
        if constexpr (tagged) {
            // The last layer's output is the step's (plain rows, read after
            // the launch); the others go out as tagged rows.
            a.out = last ? f.output : nullptr;
            a.tout = last ? nullptr : tagged_rows(f, layer, ROWS_X);
            a.tres = tagged_rows(f, layer, ROWS_R);
        } else {
            a.out = layer_output(f, layer);
            a.residual = act_rows(f, layer, 1);
        }
        gemm_split_task<EPI_RESIDUAL, Q8>(
            a, index, tile, lds,
            TracedWait{wait_for(f, layer, tile, PGPU_FLOW_MLP_IN, PGPU_FLOW_MLP_IN_TASKS), &f});
        if constexpr (tagged)
            trace_mark(f, 2);
        else
            flow_signal(f, phase_counter(f, layer, tile, PGPU_FLOW_MLP_OUT));
        break;
    }
    default:
        break;
    }
}

// Two 512-thread work-groups per CU: the projection tasks' registers and
// 49 KB of LDS (the prologue's operand buffer) set the occupancy.
template <bool Q8, int MODE, bool PRE, int R>
__global__ __launch_bounds__(kTaskThreads) void k_flow_step(pgpu_flow_step f, pgpu_paged_kv kv) {
    __shared__ uint4 lds4[kTaskLds / 8];
    flow_step_task<Q8, MODE, PRE, R>(f, kv, lds4);
}

// One kernel per (hand-off mode, prefill or decode, splits per attention
// task): each resolves its branches at compile time and carries no other
// variant's registers.
template <bool Q8, bool PRE, int R>
void launch_step(const pgpu_flow_step *step, const pgpu_paged_kv *kv, hipStream_t stream) {
    auto kernel = step->tagged == PGPU_FLOW_HANDOFF_TAGGED      ? k_flow_step<Q8, 1, PRE, R>
                  : step->tagged == PGPU_FLOW_HANDOFF_PARTS     ? k_flow_step<Q8, 2, PRE, R>
                  : step->tagged == PGPU_FLOW_HANDOFF_MERGE_OUT ? k_flow_step<Q8, 3, PRE, R>
                  : step->tagged == PGPU_FLOW_HANDOFF_FUSED_MLP
                      // decode only (pgpu_flow_launch rejects a fused prefill)
                      ? k_flow_step<Q8, PRE ? 3 : 4, PRE, R>
                      : k_flow_step<Q8, 0, PRE, R>;
    hipLaunchKernelGGL(kernel, dim3(step->tasks), dim3(kTaskThreads), 0, stream, *step, *kv);
}

template <bool Q8, bool PRE>
void launch_rounds(const pgpu_flow_step *step, const pgpu_paged_kv *kv, hipStream_t stream) {
    static_assert(PGPU_FLOW_ATTN_ROUNDS == 2, "one kernel per rounds value");
    if (step->attn_rounds == 1)
        launch_step<Q8, PRE, 1>(step, kv, stream);
    else
        launch_step<Q8, PRE, 2>(step, kv, stream);
}

}  // namespace
}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_flow_launch(void *stream, const pgpu_flow_step *step,
                                const pgpu_paged_kv *kv) {
    if (!step || !kv || !step->layers || step->layer_count <= 0 || step->layer_count > 64 ||
        step->streams <= 0 || step->tiles != (step->streams + 15) / 16 || step->tiles > 256 ||
        !step->input || !step->output || !step->act || !step->hidden || !step->part_acc ||
        !step->part_ml || step->max_splits <= 0 || step->max_splits > 255 ||
        step->ml_group < 2 * step->max_splits || step->ml_group % 32 || !step->tables ||
        !step->positions || step->table_stride <= 0 || !step->rope || !step->schedule ||
        !step->tasks || !step->phase || !step->split_done || !step->status ||
        step->attn_rounds < 1 || step->attn_rounds > PGPU_FLOW_ATTN_ROUNDS ||
        step->tagged < PGPU_FLOW_HANDOFF_COUNTER || step->tagged > PGPU_FLOW_HANDOFF_FUSED_MLP ||
        (step->tagged == PGPU_FLOW_HANDOFF_FUSED_MLP &&
         (step->prefill || step->tiles != 1 || step->streams > PGPU_FLOW_FUSED_MAX_STREAMS ||
          !step->mlp_parts)) ||
        (step->tagged != PGPU_FLOW_HANDOFF_COUNTER &&
         (!step->parts || !step->tag || step->max_splits > 32)) ||
        step->pos_delta < 0 || step->clear_words % 4 ||
        (step->clear_words && (!step->clear || (step->clear_words + PGPU_FLOW_CLEAR_WORDS - 1) /
                                                       PGPU_FLOW_CLEAR_WORDS > step->tasks)) ||
        ((step->tagged == PGPU_FLOW_HANDOFF_TAGGED || step->tagged == PGPU_FLOW_HANDOFF_MERGE_OUT ||
          step->tagged == PGPU_FLOW_HANDOFF_FUSED_MLP) && !step->rows) ||
        step->pool_offset < 0 || step->pool_offset + step->layer_count > kv->layers)
        return bad_arguments("pgpu_flow_launch");
    if (step->prefill) {
        if (step->q8)
            launch_rounds<true, true>(step, kv, (hipStream_t)stream);
        else
            launch_rounds<false, true>(step, kv, (hipStream_t)stream);
    } else if (step->q8) {
        launch_rounds<true, false>(step, kv, (hipStream_t)stream);
    } else {
        launch_rounds<false, false>(step, kv, (hipStream_t)stream);
    }
    return launch_ok("pgpu_flow_launch");
}
