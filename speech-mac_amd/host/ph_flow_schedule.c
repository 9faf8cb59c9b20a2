/* Task list of the one-launch decode step (pgpu_flow_launch, phonon_gpu.h).
 *
 * The order is the launch's dispatch order. Every task comes after the
 * tasks it waits for, so the lowest-numbered unfinished task can always run
 * and the launch cannot deadlock.
 *
 * Within that constraint the list is laid out on a model clock: attention
 * tasks advance the clock by unit_us each (they stream K/V from HBM at a
 * steady rate), and each projection phase of a tile's chain is listed
 * after_us[phase] after the tile's last attention task, i.e. about when its
 * inputs will be ready. A task listed too early holds a work-group slot
 * while it waits; one listed too late delays its chain. The next layer's
 * attention of a tile is never listed before that tile's QKV (a pending
 * chain is flushed first). */
#include "ph_internal.h"

#include <stdlib.h>

typedef struct {
    double at;        /* model time of the entry */
    size_t seq;       /* insertion order (ties) */
    uint32_t kind, layer, tile;
} Pending;

typedef struct {
    Pending *items;
    size_t count, seq;
    int fused;  /* fused MLP: MLP_OUT only after the last layer */
} Queue;

static const uint32_t kChainKinds[4] = {PGPU_FLOW_OUT, PGPU_FLOW_MLP_IN, PGPU_FLOW_MLP_OUT,
                                        PGPU_FLOW_QKV};

/* Tasks of one phase of a (layer, tile); with the fused MLP, MLP_OUT is the
 * last layer's output tasks. */
static uint32_t phase_tasks(uint32_t kind, int fused) {
    switch (kind) {
    case PGPU_FLOW_QKV: return PGPU_FLOW_QKV_TASKS;
    case PGPU_FLOW_OUT: return PGPU_FLOW_OUT_TASKS;
    case PGPU_FLOW_MLP_IN: return PGPU_FLOW_MLP_IN_TASKS;
    default: return fused ? PGPU_FLOW_FUSED_OUT_TASKS : PGPU_FLOW_MLP_OUT_TASKS;
    }
}

/* QKV tasks head by head (q, k, v of head 0, then of head 1, ...): the
 * attention of a head waits only for its own three. */
static void emit_phase(uint32_t *d, size_t *k, uint32_t kind, uint32_t layer, uint32_t tile,
                       int fused) {
    const uint32_t n = phase_tasks(kind, fused);
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t index = kind == PGPU_FLOW_QKV ? (i % 3) * PH_HEADS + i / 3 : i;
        d[(*k)++] = PGPU_FLOW_TASK(kind, layer, tile, index);
    }
}

/* Sorted insert by (at, seq). */
static void push(Queue *q, double at, uint32_t kind, uint32_t layer, uint32_t tile) {
    size_t i = q->count++;
    const Pending e = {at, q->seq++, kind, layer, tile};
    while (i > 0 && q->items[i - 1].at > at) {
        q->items[i] = q->items[i - 1];
        i--;
    }
    q->items[i] = e;
}

static void remove_at(Queue *q, size_t i) {
    for (; i + 1 < q->count; i++)
        q->items[i] = q->items[i + 1];
    q->count--;
}

/* Emits every pending entry, one kind after another (all OUT, then all
 * MLP_IN, ...): with many tiles a tile-major chain would fill the dispatch
 * window with tasks that wait for each other. */
static void flush_by_phase(Queue *q, uint32_t *d, size_t *k) {
    for (int p = 0; p < 4; p++)
        for (size_t i = 0; i < q->count;) {
            const Pending e = q->items[i];
            if (e.kind == kChainKinds[p]) {
                emit_phase(d, k, e.kind, e.layer, e.tile, q->fused);
                remove_at(q, i);
            } else {
                i++;
            }
        }
}

/* Emits every pending entry of `tile` (all tiles if tile < 0), in order. */
static void flush(Queue *q, int tile, uint32_t *d, size_t *k) {
    for (size_t i = 0; i < q->count;) {
        const Pending e = q->items[i];
        if (tile < 0 || e.tile == (uint32_t)tile) {
            emit_phase(d, k, e.kind, e.layer, e.tile, q->fused);
            remove_at(q, i);
        } else {
            i++;
        }
    }
}

pgpu_flow_placement ph_flow_default_placement(int rounds) {
    /* Clock in ATTN tasks (rounds 256-key splits, 128 KB of K/V each): at
     * B = 64 a 16-stream tile's attention is ~640 splits. Swept on MI355X
     * at B = 64 (one split per task) and B = 48, 96, 128, 160 (two). */
    const pgpu_flow_placement one = {1.0f, {550.0f, 1000.0f, 1450.0f, 1750.0f}};
    const pgpu_flow_placement two = {2.0f, {1150.0f, 1850.0f, 2550.0f, 3050.0f}};
    return rounds > 1 ? two : one;
}

size_t pgpu_flow_schedule(size_t streams, size_t layers, const size_t *units,
                          const pgpu_flow_placement *place, int flags, uint32_t *schedule,
                          size_t capacity) {
    if (!streams || !layers || !units || (flags & ~(PGPU_FLOW_SCHEDULE_PREFILL |
                                                    PGPU_FLOW_SCHEDULE_FUSED_MLP)))
        return 0;
    const int prefill = (flags & PGPU_FLOW_SCHEDULE_PREFILL) != 0;
    const int fused = !prefill && (flags & PGPU_FLOW_SCHEDULE_FUSED_MLP) != 0;
    const size_t tiles = (streams + 15) / 16;
    size_t attn = 0;
    for (size_t s = 0; s < streams; s++)
        attn += units[s];
    const size_t chain = PGPU_FLOW_QKV_TASKS + PGPU_FLOW_OUT_TASKS + PGPU_FLOW_MLP_IN_TASKS;
    const size_t tasks = layers * tiles * chain +
                         (fused ? tiles * PGPU_FLOW_FUSED_OUT_TASKS
                                : layers * tiles * PGPU_FLOW_MLP_OUT_TASKS) +
                         layers * PH_HEADS * attn;
    if (!schedule || capacity < tasks)
        return tasks;
    double after[4] = {0.0, 0.0, 0.0, 0.0}, unit_us = 0.0;
    if (place && !prefill) {
        unit_us = place->unit_us > 0.0f ? place->unit_us : 0.0;
        for (int p = 0; p < 4; p++) {
            const double a = place->after_us[p] > 0.0f ? place->after_us[p] : 0.0;
            after[p] = p && a < after[p - 1] ? after[p - 1] : a;  /* phases in order */
        }
    }
    Queue q = {malloc(4 * tiles * sizeof(Pending)), 0, 0, fused};
    if (!q.items)
        return 0;
    uint32_t *d = schedule;
    size_t k = 0;
    for (size_t t = 0; t < tiles; t++)
        emit_phase(d, &k, PGPU_FLOW_QKV, 0, (uint32_t)t, fused);
    double now = 0.0;
    for (size_t l = 0; l < layers; l++) {
        /* With prefill every ATTN task of layer l waits for the QKV of all
         * tiles: everything pending goes first, phase by phase. */
        if (prefill)
            flush_by_phase(&q, d, &k);
        for (size_t t = 0; t < tiles; t++) {
            flush(&q, (int)t, d, &k);  /* tile t's chain, through its QKV of layer l */
            for (size_t n = 0; n < 16 && t * 16 + n < streams; n++)
                for (size_t j = 0; j < units[t * 16 + n]; j++)
                    for (uint32_t h = 0; h < PH_HEADS; h++) {
                        while (q.count && q.items[0].at <= now) {
                            emit_phase(d, &k, q.items[0].kind, q.items[0].layer,
                                       q.items[0].tile, fused);
                            remove_at(&q, 0);
                        }
                        d[k++] = PGPU_FLOW_TASK(PGPU_FLOW_ATTN, l, t, h | j << 3 | n << 11);
                        now += unit_us;
                    }
            for (int p = 0; p < 4; p++) {
                if (p == 3 && l + 1 == layers)
                    break;
                if (p == 2 && fused && l + 1 < layers)
                    continue; /* the next layer's QKV tasks sum the MLP partials */
                /* prefill: the layer's chains wait for the next layer's flush */
                push(&q, prefill ? 1e300 : now + after[p], kChainKinds[p],
                     (uint32_t)(p == 3 ? l + 1 : l), (uint32_t)t);
            }
        }
    }
    if (prefill)
        flush_by_phase(&q, d, &k);
    else
        flush(&q, -1, d, &k);
    free(q.items);
    return k;
}
