/* Batched Flow decode step over a paged KV pool (phonon_flow_batch.h).
 *
 * One step of B streams runs five kernels per layer
 * (src/phonon_transformer.c:406-453):
 *   LN1 + QKV projection + RoPE + append      pgpu_gemm_qkv
 *   split attention over the pool (partials)  pgpu_attention
 *   split merge + out projection + residual   pgpu_gemm_residual
 *   LN2 + MLP in projection + GELU            pgpu_gemm_gelu_split
 *   MLP out projection + residual             pgpu_gemm_residual
 * then advances every stream's position on the device. */
#include "ph_internal.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

struct PhononFlowModel {
    size_t layers;
    pgpu_matrix *qkv, *out, *mlp_in, *mlp_out;
    pgpu_wide_matrix *wide;       /* [layers][4]: the prefill projections' weights */
    float *norms; /* dev [layers][4][512]: norm1 w, b, norm2 w, b */
    pgpu_flow_layer *flow_layers; /* dev [layers]: operands of the one-launch step */
    int q8;                       /* 1/0: every matrix Q8/BF16; -1: mixed */
    void **allocations;
    size_t allocation_count, device_bytes;
};

struct PhononKvPool {
    pgpu_paged_kv kv;
    int32_t *free_ids;
    size_t free_count;
    unsigned char *in_use;
};

struct PhononFlowBatch {
    const PhononFlowModel *model;
    PhononKvPool *pool;
    size_t max_streams, padded_streams, max_positions, table_len, max_splits, streams;
    size_t splits; /* attention splits of the work being enqueued (<= max_splits) */
    void *stream;
    float *x, *r, *q, *in, *out, *rows;
    uint16_t *xh; /* split fragments of the MLP hidden rows */
    int32_t *positions, *tables;
    const int32_t *table_src, *table_map; /* a prefill call's uploads (in pre.stage_dev) */
    struct {
        int active;                 /* the streams are a prefill's pseudo-streams */
        int exact;                  /* attention with the decode step's arithmetic */
        const int32_t *entries;     /* (dev) [count][4]: work entries of pgpu_prefill_attention */
        int32_t *host;              /* [cap][4] */
        size_t count, cap;
        const int32_t *runs;        /* (dev) [runs_count][2]: the run-based prefill attentions */
        int32_t *runs_host;
        size_t runs_count, runs_cap;
        const int32_t *pairs;       /* (dev) [pairs_count][4]: runs paired per stream (mfma) */
        int32_t *pairs_host;
        size_t pairs_count, pairs_cap;
        uint16_t *split;            /* (dev) split fragments [max_streams/16][16][1536] */
        unsigned char *stage;       /* pinned host staging of a prefill call's uploads */
        unsigned char *stage_dev;   /* (dev) the same layout: one copy moves the whole area */
        size_t stage_cap, stage_used;
    } pre;
    int flow;                       /* 1: one launch per step (pgpu_flow_launch) */
    struct {
        size_t cap, cap_layers;     /* padded streams and layers the buffers hold */
        float *act, *part_acc, *part_ml;
        uint16_t *hidden;
        unsigned *counters;         /* two sets of counter_words: the next step's set is
                                       all zero (the step before zeroes it) */
        size_t counter_words;
        int parity;                 /* the set the next step uses */
        uint64_t *rows, *parts;     /* (dev) tagged mode's hand-off words (pgpu_flow_step) */
        size_t rows_words, parts_words;
        float *mlp_parts;           /* (dev) fused MLP's partials, made on first use */
        size_t mlp_words;
        uint32_t tag;               /* tagged mode's tag of the next step, never 0 */
        int tagged_set;             /* -1: by batch size, else the caller's choice */
        uint32_t *schedule, *host_schedule;
        size_t schedule_cap, host_cap, tasks;
        size_t *cover;              /* [max_streams] splits the schedule lists per stream */
        size_t *units;              /* [max_streams] ATTN tasks per (stream, head) for them */
        int rounds;                 /* splits per ATTN task the schedule was built for */
        int rounds_set;             /* 0: by batch size, else the caller's choice */
        int place_set;              /* the caller set the placement */
        size_t streams, layers;     /* what the schedule was built for (0: none) */
        int prefill, fused;
        unsigned version;           /* bumped by every rebuild */
        pgpu_flow_placement place;  /* chain placement in the task list */
        uint64_t *trace;            /* (dev) optional task timeline, trace_cap tasks */
        size_t trace_cap;
        unsigned wait_us;           /* give-up bound of the tasks' waits (0: 1 s) */
    } fl;
    int *status;
    pgpu_attention_scratch scratch;
    size_t *host_positions;
    int pos_lag;                    /* one-launch steps the device positions trail
                                       host_positions by (pgpu_flow_step.pos_delta) */
    /* Captured steps, keyed by what the capture baked in. Two entries, so a
     * caller that alternates two buffers (output feeding the next input)
     * replays both without capturing again. */
    struct {
        void *exec;
        size_t streams, splits;
        float theta;
        const float *input;
        float *output;
    } graphs[2];
    size_t graph_victim;
    int eager;                         /* launch kernels directly, no graph */
    void *time_before, *time_after;    /* events around the next step's kernels, or NULL */
    size_t groups;                     /* stream groups run concurrently */
    void *side[PH_MAX_GROUPS - 1];     /* HIP streams of groups 1.. */
    void *fork, *join[PH_MAX_GROUPS - 1];
};

/* ---------------------------------------------------------------- model -- */

void phonon_flow_model_destroy(PhononFlowModel *model) {
    if (!model)
        return;
    if (model->allocation_count)
        (void)pgpu_stream_sync(ph_stream());
    for (size_t i = 0; i < model->allocation_count; i++)
        pgpu_free(model->allocations[i]);
    free(model->allocations);
    free(model->qkv);
    free(model->out);
    free(model->mlp_in);
    free(model->mlp_out);
    free(model->wide);
    free(model);
}

int phonon_flow_model_create(const PhononFlowLayerWeights *weights, size_t layers,
                             PhononFlowModel **model) {
    if (!model)
        return 0;
    *model = NULL;
    if (!weights || !layers || layers > 64 || !ph_init())
        return 0;
    PhononFlowModel *m = calloc(1, sizeof(*m));
    if (!m)
        return 0;
    m->layers = layers;
    m->qkv = calloc(layers, sizeof(pgpu_matrix));
    m->out = calloc(layers, sizeof(pgpu_matrix));
    m->mlp_in = calloc(layers, sizeof(pgpu_matrix));
    m->mlp_out = calloc(layers, sizeof(pgpu_matrix));
    m->wide = calloc(layers * 4, sizeof(pgpu_wide_matrix));
    /* Per layer 4 uploads and up to 4 x 3 prefill copies; norms; table. */
    m->allocations = calloc(layers * 16 + 2, sizeof(void *));
    float *norms = malloc(layers * 4 * PH_WIDTH * sizeof(float));
    int ok = m->qkv && m->out && m->mlp_in && m->mlp_out && m->wide && m->allocations && norms;
    for (size_t l = 0; ok && l < layers; l++) {
        const PhononFlowLayerWeights *w = &weights[l];
        struct {
            const PhononTensorView *view;
            size_t rows, columns;
            pgpu_matrix *dst;
        } mats[4] = {{w->qkv, 3 * PH_WIDTH, PH_WIDTH, &m->qkv[l]},
                     {w->attention_out, PH_WIDTH, PH_WIDTH, &m->out[l]},
                     {w->mlp_in, PH_FFN, PH_WIDTH, &m->mlp_in[l]},
                     {w->mlp_out, PH_WIDTH, PH_FFN, &m->mlp_out[l]}};
        for (int i = 0; ok && i < 4; i++) {
            void *dev = NULL;
            ok = ph_matrix_upload(mats[i].view, mats[i].rows, mats[i].columns, mats[i].dst, &dev);
            if (ok) {
                m->allocations[m->allocation_count++] = dev;
                m->device_bytes += mats[i].dst->rows * mats[i].dst->columns *
                                   (mats[i].dst->q8 ? 1 : 2) +
                                   (mats[i].dst->q8 ? mats[i].dst->rows * mats[i].dst->columns / 16 : 0);
            }
            /* The batched prefill's projections read bf16 or fp16 fragments
             * (and fp32 scales): converted once here from Q8 (exact). */
            pgpu_wide_matrix *wide = &m->wide[l * 4 + i];
            const pgpu_matrix *mat = mats[i].dst;
            wide->rows = mat->rows;
            wide->columns = mat->columns;
            if (ok && !mat->q8) {
                wide->values = mat->values;
            } else if (ok) {
                const size_t n = mat->rows * mat->columns;
                uint16_t *values = pgpu_malloc(n * sizeof(uint16_t));
                float *scales = values ? pgpu_malloc(n / 32 * sizeof(float)) : NULL;
                uint16_t *f16 = scales ? pgpu_malloc(n * sizeof(uint16_t)) : NULL;
                if (values)
                    m->allocations[m->allocation_count++] = values;
                if (scales)
                    m->allocations[m->allocation_count++] = scales;
                if (f16)
                    m->allocations[m->allocation_count++] = f16;
                ok = f16 && pgpu_wide_from_matrix(ph_stream(), mat, values, scales, f16);
                wide->values = values;
                wide->scales = scales;
                wide->values_f16 = f16;
                m->device_bytes += 2 * n * sizeof(uint16_t) + n / 32 * sizeof(float);
            }
        }
        float *n = norms + l * 4 * PH_WIDTH;
        ok = ok && ph_vector_decode(w->norm1_weight, PH_WIDTH, n) &&
             ph_vector_decode(w->norm1_bias, PH_WIDTH, n + PH_WIDTH) &&
             ph_vector_decode(w->norm2_weight, PH_WIDTH, n + 2 * PH_WIDTH) &&
             ph_vector_decode(w->norm2_bias, PH_WIDTH, n + 3 * PH_WIDTH);
    }
    if (ok) {
        m->norms = pgpu_malloc(layers * 4 * PH_WIDTH * sizeof(float));
        ok = m->norms != NULL;
        if (ok) {
            m->allocations[m->allocation_count++] = m->norms;
            ok = pgpu_copy_h2d(ph_stream(), m->norms, norms, layers * 4 * PH_WIDTH * sizeof(float));
        }
    }
    free(norms);
    /* Operand table of the one-launch step (pgpu_flow_launch). */
    pgpu_flow_layer *table = ok ? calloc(layers, sizeof(pgpu_flow_layer)) : NULL;
    ok = ok && table;
    m->q8 = ok ? m->qkv[0].q8 : 0;
    for (size_t l = 0; ok && l < layers; l++) {
        const pgpu_matrix *mats[4] = {&m->qkv[l], &m->out[l], &m->mlp_in[l], &m->mlp_out[l]};
        for (int i = 0; i < 4; i++) {
            table[l].values[i] = mats[i]->values;
            table[l].scales[i] = mats[i]->scales;
            if (mats[i]->q8 != m->q8)
                m->q8 = -1;
        }
        table[l].norms = m->norms + l * 4 * PH_WIDTH;
    }
    if (ok) {
        m->flow_layers = pgpu_malloc(layers * sizeof(pgpu_flow_layer));
        ok = m->flow_layers != NULL;
        if (ok) {
            m->allocations[m->allocation_count++] = m->flow_layers;
            ok = pgpu_copy_h2d(ph_stream(), m->flow_layers, table,
                               layers * sizeof(pgpu_flow_layer));
        }
    }
    free(table);
    if (!ok) {
        phonon_flow_model_destroy(m);
        return 0;
    }
    *model = m;
    return 1;
}

size_t phonon_flow_model_layers(const PhononFlowModel *model) {
    return model ? model->layers : 0;
}

size_t phonon_flow_model_device_bytes(const PhononFlowModel *model) {
    return model ? model->device_bytes : 0;
}

/* ----------------------------------------------------------------- pool -- */

int phonon_kv_pool_create(size_t layers, size_t blocks, PhononKvPool **pool) {
    if (!pool)
        return 0;
    *pool = NULL;
    const size_t block_floats = (size_t)PH_HEADS * 2 * 16 * PH_HEAD;
    if (!layers || layers > 64 || !blocks || blocks > INT32_MAX ||
        blocks > SIZE_MAX / (layers * block_floats * sizeof(float)) || !ph_init())
        return 0;
    PhononKvPool *p = calloc(1, sizeof(*p));
    if (!p)
        return 0;
    p->kv.layers = (int)layers;
    p->kv.blocks = blocks;
    p->kv.layer_stride = blocks * block_floats;
    p->kv.base = pgpu_malloc(layers * p->kv.layer_stride * sizeof(float));
    p->free_ids = malloc(blocks * sizeof(int32_t));
    p->in_use = calloc(blocks, 1);
    /* Zeroed so that never-written slots read as finite values. */
    if (!p->kv.base || !p->free_ids || !p->in_use ||
        !pgpu_memset(ph_stream(), p->kv.base, 0, layers * p->kv.layer_stride * sizeof(float)) ||
        !pgpu_stream_sync(ph_stream())) {
        phonon_kv_pool_destroy(p);
        return 0;
    }
    /* Hand out low ids first. */
    for (size_t i = 0; i < blocks; i++)
        p->free_ids[i] = (int32_t)(blocks - 1 - i);
    p->free_count = blocks;
    *pool = p;
    return 1;
}

void phonon_kv_pool_destroy(PhononKvPool *pool) {
    if (!pool)
        return;
    if (pool->kv.base) {
        (void)pgpu_stream_sync(ph_stream());
        pgpu_free(pool->kv.base);
    }
    free(pool->free_ids);
    free(pool->in_use);
    free(pool);
}

size_t phonon_kv_pool_free_blocks(const PhononKvPool *pool) {
    return pool ? pool->free_count : 0;
}

int phonon_kv_pool_alloc(PhononKvPool *pool, size_t count, int32_t *blocks) {
    if (!pool || (count && !blocks) || count > pool->free_count)
        return 0;
    for (size_t i = 0; i < count; i++) {
        blocks[i] = pool->free_ids[--pool->free_count];
        pool->in_use[blocks[i]] = 1;
    }
    return 1;
}

int phonon_kv_pool_release(PhononKvPool *pool, size_t count, const int32_t *blocks) {
    if (!pool || (count && !blocks))
        return 0;
    for (size_t i = 0; i < count; i++)
        if (blocks[i] < 0 || (size_t)blocks[i] >= pool->kv.blocks || !pool->in_use[blocks[i]])
            return 0;
    for (size_t i = 0; i < count; i++) {
        pool->in_use[blocks[i]] = 0;
        pool->free_ids[pool->free_count++] = blocks[i];
    }
    return 1;
}

int phonon_kv_pool_fill_normal(PhononKvPool *pool, uint64_t seed) {
    if (!pool)
        return 0;
    return pgpu_fill_normal(ph_stream(), pool->kv.base, pool->kv.layers * pool->kv.layer_stride,
                            seed) &&
           pgpu_stream_sync(ph_stream());
}

const pgpu_paged_kv *ph_pool_kv(const PhononKvPool *pool) { return &pool->kv; }

int phonon_kv_pool_view(const PhononKvPool *pool, pgpu_paged_kv *view) {
    if (!pool || !view)
        return 0;
    *view = pool->kv;
    return 1;
}

static int pool_copy(const PhononKvPool *pool, const int32_t *table, size_t table_len,
                     size_t first, size_t count, float *keys, float *values, size_t capacity,
                     int to_host) {
    if (!pool || !table || !keys || !values || !count || first + count > capacity ||
        first + count > table_len * 16 || capacity > PHONON_FLOW_MAX_POSITIONS)
        return 0;
    for (size_t i = first / 16; i < (first + count + 15) / 16; i++)
        if (table[i] < 0 || (size_t)table[i] >= pool->kv.blocks)
            return 0;
    /* Device staging holds only the requested rows, [layer][count][512]. */
    const size_t layers = (size_t)pool->kv.layers;
    const size_t row_bytes = count * PH_WIDTH * sizeof(float);
    const size_t bytes = layers * row_bytes;
    void *stream = ph_stream();
    float *dk = pgpu_malloc(bytes), *dv = pgpu_malloc(bytes);
    int32_t *dt = pgpu_malloc(table_len * sizeof(int32_t));
    int *status = pgpu_malloc(sizeof(int));
    int ok = dk && dv && dt && status && pgpu_memset(stream, status, 0, sizeof(int)) &&
             pgpu_copy_h2d(stream, dt, table, table_len * sizeof(int32_t));
    for (size_t l = 0; ok && !to_host && l < layers; l++) {
        const size_t host = (l * capacity + first) * PH_WIDTH, dev = l * count * PH_WIDTH;
        ok = pgpu_copy_h2d(stream, dk + dev, keys + host, row_bytes) &&
             pgpu_copy_h2d(stream, dv + dev, values + host, row_bytes);
    }
    ok = ok && pgpu_kv_copy(stream, &pool->kv, dt, (int)first, (int)count, 0, (int)layers, dk,
                            dv, count, to_host, status);
    int st = 1;
    ok = ok && pgpu_copy_d2h(stream, &st, status, sizeof(int)) && st == 0;
    for (size_t l = 0; ok && to_host && l < layers; l++) {
        const size_t host = (l * capacity + first) * PH_WIDTH, dev = l * count * PH_WIDTH;
        ok = pgpu_copy_d2h(stream, keys + host, dk + dev, row_bytes) &&
             pgpu_copy_d2h(stream, values + host, dv + dev, row_bytes);
    }
    (void)pgpu_stream_sync(stream);
    pgpu_free(dk);
    pgpu_free(dv);
    pgpu_free(dt);
    pgpu_free(status);
    return ok;
}

int phonon_kv_pool_write(PhononKvPool *pool, const int32_t *table, size_t table_len,
                         size_t first, size_t count, const float *keys, const float *values,
                         size_t capacity) {
    return pool_copy(pool, table, table_len, first, count, (float *)keys, (float *)values,
                     capacity, 0);
}

int phonon_kv_pool_read(const PhononKvPool *pool, const int32_t *table, size_t table_len,
                        size_t first, size_t count, float *keys, float *values,
                        size_t capacity) {
    return pool_copy(pool, table, table_len, first, count, keys, values, capacity, 1);
}

/* ---------------------------------------------------------------- batch -- */

static void drop_graphs(PhononFlowBatch *b) {
    for (size_t i = 0; i < 2; i++) {
        pgpu_graph_destroy(b->graphs[i].exec);
        b->graphs[i].exec = NULL;
    }
}

void phonon_flow_batch_destroy(PhononFlowBatch *b) {
    if (!b)
        return;
    if (b->stream)
        (void)pgpu_stream_sync(b->stream);
    drop_graphs(b);
    for (size_t g = 0; g + 1 < PH_MAX_GROUPS; g++) {
        if (b->side[g])
            (void)pgpu_stream_sync(b->side[g]);
        pgpu_stream_destroy(b->side[g]);
        pgpu_event_destroy(b->join[g]);
    }
    pgpu_event_destroy(b->fork);
    void *bufs[] = {b->x,    b->r,  b->q,         b->in,     b->out,
                    b->rows, b->xh, b->positions, b->tables, b->status,
                    b->scratch.part_acc, b->scratch.part_ml, b->pre.stage_dev,
                    b->fl.act, b->fl.part_acc, b->fl.part_ml, b->fl.hidden, b->fl.counters,
                    b->fl.rows, b->fl.parts, b->fl.mlp_parts, b->fl.schedule};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
        pgpu_free(bufs[i]);
    pgpu_stream_destroy(b->stream);
    free(b->pre.host);
    pgpu_host_free(b->pre.stage);
    free(b->pre.runs_host);
    free(b->pre.pairs_host);
    pgpu_free(b->pre.split);
    free(b->host_positions);
    free(b->fl.host_schedule);
    free(b->fl.cover);
    free(b->fl.units);
    free(b);
}

int phonon_flow_batch_create(const PhononFlowModel *model, PhononKvPool *pool,
                             size_t max_streams, size_t max_positions, PhononFlowBatch **batch) {
    if (!batch)
        return 0;
    *batch = NULL;
    if (!model || !pool || !max_streams || max_streams > 4096 || !max_positions ||
        max_positions > PHONON_FLOW_MAX_POSITIONS || (size_t)pool->kv.layers < model->layers ||
        !ph_init())
        return 0;
    PhononFlowBatch *b = calloc(1, sizeof(*b));
    if (!b)
        return 0;
    b->model = model;
    b->pool = pool;
    b->fl.tagged_set = -1;
    b->max_streams = max_streams;
    b->padded_streams = (max_streams + 15) / 16 * 16;
    b->max_positions = max_positions;
    b->table_len = (max_positions + 15) / 16;
    b->max_splits = (max_positions + PH_SPLIT_KEYS - 1) / PH_SPLIT_KEYS;
    const size_t rows = b->padded_streams * PH_WIDTH * sizeof(float);
    const size_t split2048 = b->padded_streams * PH_FFN * 3 * sizeof(uint16_t);
    const size_t slots = max_streams * PH_HEADS * b->max_splits;
    b->groups = PH_DEFAULT_GROUPS;
    b->flow = 1;
    b->fl.place = ph_flow_default_placement(1);
    /* One HIP stream; the side streams of stream groups are made when groups
     * are asked for (phonon_flow_batch_set_groups), so a batch per request
     * holds one stream and requests on separate caches spread over the
     * GPU's hardware queues. */
    int ok = pgpu_stream_create(&b->stream);
    b->x = pgpu_malloc(rows);
    b->r = pgpu_malloc(rows);
    b->q = pgpu_malloc(rows);
    b->in = pgpu_malloc(rows);
    b->out = pgpu_malloc(rows);
    b->rows = pgpu_malloc(2 * (size_t)pool->kv.layers * PH_WIDTH * sizeof(float));
    b->xh = pgpu_malloc(split2048);
    b->positions = pgpu_malloc(b->padded_streams * sizeof(int32_t));
    b->tables = pgpu_malloc(max_streams * b->table_len * sizeof(int32_t));
    b->status = pgpu_malloc(sizeof(int));
    b->scratch.part_acc = pgpu_malloc(slots * 64 * sizeof(float));
    b->scratch.part_ml = pgpu_malloc(slots * 2 * sizeof(float));
    b->scratch.max_streams = (int)max_streams;
    b->scratch.max_splits = (int)b->max_splits;
    b->host_positions = calloc(max_streams, sizeof(size_t));
    b->fl.cover = calloc(max_streams, sizeof(size_t));
    b->fl.units = calloc(max_streams, sizeof(size_t));
    ok = ok && b->x && b->r && b->q && b->in && b->out && b->rows && b->xh && b->positions &&
         b->tables && b->status && b->scratch.part_acc && b->scratch.part_ml &&
         b->host_positions && b->fl.cover && b->fl.units;
    /* Zero everything a kernel may read before writing (padding streams of the
     * split fragments, positions, status). */
    ok = ok && pgpu_memset(b->stream, b->xh, 0, split2048) &&
         pgpu_memset(b->stream, b->positions, 0, b->padded_streams * sizeof(int32_t)) &&
         pgpu_memset(b->stream, b->tables, 0, max_streams * b->table_len * sizeof(int32_t)) &&
         pgpu_memset(b->stream, b->status, 0, sizeof(int)) &&
         pgpu_memset(b->stream, b->x, 0, rows) && pgpu_memset(b->stream, b->in, 0, rows) &&
         pgpu_stream_sync(b->stream);
    if (!ok) {
        phonon_flow_batch_destroy(b);
        return 0;
    }
    *batch = b;
    return 1;
}

int phonon_flow_batch_set_streams(PhononFlowBatch *b, size_t streams, const size_t *positions,
                                  const int32_t *tables, size_t table_len) {
    if (!b || !streams || streams > b->max_streams || !positions || !tables ||
        table_len != b->table_len)
        return 0;
    int32_t *pos32 = malloc(streams * sizeof(int32_t));
    if (!pos32)
        return 0;
    for (size_t s = 0; s < streams; s++) {
        if (positions[s] >= b->max_positions) {
            free(pos32);
            return 0;
        }
        pos32[s] = (int32_t)positions[s];
    }
    int ok = pgpu_stream_sync(b->stream) &&
             pgpu_copy_h2d(b->stream, b->positions, pos32, streams * sizeof(int32_t)) &&
             pgpu_copy_h2d(b->stream, b->tables, tables, streams * table_len * sizeof(int32_t));
    free(pos32);
    if (!ok)
        return 0;
    memcpy(b->host_positions, positions, streams * sizeof(size_t));
    b->pos_lag = 0;
    b->streams = streams;
    b->pre.active = 0;
    return 1;
}

int ph_batch_bind_model(PhononFlowBatch *b, const PhononFlowModel *model) {
    if (!b || !model || model->layers > (size_t)b->pool->kv.layers)
        return 0;
    if (b->model != model) {
        drop_graphs(b);
        b->model = model;
    }
    return 1;
}

int ph_batch_set_single(PhononFlowBatch *b, size_t position, const int32_t *table_dev) {
    int32_t p = (int32_t)position;
    if (!pgpu_copy_h2d(b->stream, b->positions, &p, sizeof(p)) ||
        !pgpu_copy_d2d(b->stream, b->tables, table_dev, b->table_len * sizeof(int32_t)))
        return 0;
    b->host_positions[0] = position;
    b->pos_lag = 0;
    b->streams = 1;
    b->pre.active = 0;
    return 1;
}

/* Brings the device positions up to host_positions: a one-launch step
 * leaves them as they are (its kernels add pos_lag), every other kernel
 * reads them as stored. */
static int fold_positions(PhononFlowBatch *b) {
    if (!b->pos_lag)
        return 1;
    if (!pgpu_advance_positions(b->stream, b->positions, (int)b->streams, b->pos_lag))
        return 0;
    b->pos_lag = 0;
    return 1;
}

/* Attention splits covering every active stream's context after `ahead`
 * more steps (capped by the batch's maximum): the attention grid and the
 * partial layout are sized by the live contexts, not by max_positions. */
static size_t splits_for(const PhononFlowBatch *b, size_t ahead) {
    size_t top = 0;
    for (size_t s = 0; s < b->streams; s++)
        if (b->host_positions[s] > top)
            top = b->host_positions[s];
    const size_t keys = top + 1 + ahead;
    const size_t splits = (keys + PH_SPLIT_KEYS - 1) / PH_SPLIT_KEYS;
    return splits < b->max_splits ? splits : b->max_splits;
}

/* Enqueues layers [first, first+count) for streams [s0, s0+n) of the batch
 * (s0 a multiple of 16) on `stream`. Every buffer is used at the group's
 * offset, so groups share no memory and may run concurrently. */
/* Layers [first, first+count) of a batched prefill (pgpu_prefill.hip): per
 * layer LayerNorm into split fragments, the large-M QKV projection (RoPE,
 * K/V append), the causal attention (fast, or exact: the decode step's
 * split partials merged by the OUT operand pass), the OUT projection, the
 * second LayerNorm, MLP_IN and MLP_OUT. */
static int enqueue_prefill(PhononFlowBatch *b, void *stream, size_t first, size_t count,
                           size_t pool_offset, const float *input, float *output,
                           const float *rope) {
    const PhononFlowModel *m = b->model;
    const int n = (int)b->streams;
    const pgpu_attention_scratch scratch = {b->scratch.part_acc, b->scratch.part_ml, n,
                                            (int)b->splits};
    uint16_t *xs = b->pre.split;
    const float *cur = input;
    /* The exact mode keeps the three bf16 split terms of each activation
     * (the projections have the bits of single steps). The fast modes take
     * two fp16 terms (22 significant bits) on the fp16 matrix cores where a
     * layer's matrices are Q8 (exact in fp16): two thirds of the work. Two
     * bf16 terms (16 significant bits) measured 10x the oracle's distance
     * from float64 at the benchmark weights over a 256-position prefill of
     * the 12-layer stack (max 0.25 vs 0.046), three terms below it
     * (0.005-0.024). */
    for (size_t l = first; l < first + count; l++) {
        const pgpu_wide_matrix *wide = &m->wide[l * 4];
        const int terms = b->pre.exact != 1 && wide[0].values_f16 && wide[1].values_f16 &&
                                  wide[2].values_f16 && wide[3].values_f16
                              ? PGPU_SPLIT_F16_PAIR
                              : 3;
        const float *norm = m->norms + l * 4 * PH_WIDTH;
        float *next = (l + 1 == first + count) ? output : b->x;
        const int layer = (int)(l + pool_offset);
        if (!pgpu_rows_split_ln(stream, cur, norm, norm + PH_WIDTH, 1e-5f, n, terms, xs,
                                b->status) ||
            !pgpu_prefill_gemm_qkv(stream, &m->wide[l * 4], xs, n, terms, &b->pool->kv, layer,
                                   b->tables,
                                   (int)b->table_len, b->positions, rope, b->q, b->status))
            return 0;
        if (!(b->pre.exact == 1
                  ? pgpu_prefill_attention(stream, b->q, &b->pool->kv, layer, b->tables,
                                           (int)b->table_len, b->positions, n, PH_HEADS,
                                           (int)b->splits, b->pre.entries, (int)b->pre.count,
                                           &scratch, b->status) &&
                        pgpu_rows_split_attention(stream, &scratch, b->positions, n,
                                                  (int)b->splits, xs, b->status)
              : b->pre.exact == 2
                  ? pgpu_prefill_attention_rows(stream, b->q, &b->pool->kv, layer, b->tables,
                                                (int)b->table_len, b->positions, n,
                                                b->pre.runs, (int)b->pre.runs_count, xs,
                                                terms, b->status)
                  : pgpu_prefill_attention_mfma(stream, b->q, &b->pool->kv, layer, b->tables,
                                                (int)b->table_len, b->positions, n,
                                                b->pre.pairs, (int)b->pre.pairs_count, xs,
                                                terms, b->status)) ||
            !pgpu_prefill_gemm_residual(stream, &m->wide[l * 4 + 1], xs, n, terms, cur, b->r,
                                        b->status) ||
            !pgpu_rows_split_ln(stream, b->r, norm + 2 * PH_WIDTH, norm + 3 * PH_WIDTH, 1e-5f,
                                n, terms, xs, b->status) ||
            !pgpu_prefill_gemm_gelu_split(stream, &m->wide[l * 4 + 2], xs, n, terms, b->xh,
                                          b->status) ||
            !pgpu_prefill_gemm_residual(stream, &m->wide[l * 4 + 3], b->xh, n, terms, b->r,
                                        next, b->status))
            return 0;
        cur = next;
    }
    return 1;
}

static int enqueue_group(PhononFlowBatch *b, void *stream, size_t s0, size_t n, size_t first,
                         size_t count, size_t pool_offset, const float *input, float *output,
                         const float *rope) {
    if (b->pre.active)
        return enqueue_prefill(b, stream, first, count, pool_offset, input, output, rope);
    const PhononFlowModel *m = b->model;
    const size_t slot0 = s0 * PH_HEADS * b->splits;
    const pgpu_attention_scratch scratch = {b->scratch.part_acc + slot0 * 64,
                                            b->scratch.part_ml + slot0 * 2, (int)n,
                                            (int)b->splits};
    float *x = b->x + s0 * PH_WIDTH, *r = b->r + s0 * PH_WIDTH, *q = b->q + s0 * PH_WIDTH;
    uint16_t *xh = b->xh + (s0 / 16) * (PH_FFN / 32) * 1536;
    const int32_t *positions = b->positions + s0, *tables = b->tables + s0 * b->table_len;
    const float *cur = input + s0 * PH_WIDTH;
    /* A layer reads its input only in the QKV prologue and the out-projection
     * residual, both before its last kernel writes `next`: in-place is safe. */
    for (size_t l = first; l < first + count; l++) {
        const float *norm = m->norms + l * 4 * PH_WIDTH;
        float *next = (l + 1 == first + count) ? output + s0 * PH_WIDTH : x;
        const int pool_layer = (int)(l + pool_offset);
        const pgpu_gemm_input ln1 = {.ln_rows = cur, .ln_weight = norm,
                                     .ln_bias = norm + PH_WIDTH, .ln_epsilon = 1e-5f};
        const pgpu_gemm_input att = {.attn_acc = scratch.part_acc,
                                     .attn_ml = scratch.part_ml,
                                     .attn_positions = positions,
                                     .attn_max_splits = (int)b->splits};
        const pgpu_gemm_input ln2 = {.ln_rows = r, .ln_weight = norm + 2 * PH_WIDTH,
                                     .ln_bias = norm + 3 * PH_WIDTH, .ln_epsilon = 1e-5f};
        const pgpu_gemm_input hidden = {.split = xh};
        if (!pgpu_gemm_qkv(stream, &m->qkv[l], &ln1, (int)n, &b->pool->kv, pool_layer, tables,
                           (int)b->table_len, positions, rope, q, b->status) ||
            !(b->pre.active
                  ? pgpu_prefill_attention(stream, q, &b->pool->kv, pool_layer, tables,
                                           (int)b->table_len, positions, (int)n, PH_HEADS,
                                           (int)b->splits, b->pre.entries, (int)b->pre.count,
                                           &scratch, b->status)
                  : pgpu_attention(stream, q, &b->pool->kv, pool_layer, tables,
                                   (int)b->table_len, positions, (int)n, PH_HEADS,
                                   (int)b->splits, &scratch, b->status)) ||
            !pgpu_gemm_residual(stream, &m->out[l], &att, (int)n, cur, r, b->status) ||
            !pgpu_gemm_gelu_split(stream, &m->mlp_in[l], &ln2, (int)n, xh, b->status) ||
            !pgpu_gemm_residual(stream, &m->mlp_out[l], &hidden, (int)n, r, next, b->status))
            return 0;
        cur = next;
    }
    return 1;
}

int ph_batch_enqueue_layers(PhononFlowBatch *b, size_t first, size_t count, size_t pool_offset,
                            const float *input, float *output, float theta) {
    if (!b->streams || first + count > b->model->layers ||
        first + count + pool_offset > (size_t)b->pool->kv.layers)
        return 0;
    const float *rope = ph_rope_table(theta);
    b->splits = splits_for(b, 0);
    return rope && fold_positions(b) &&
           enqueue_group(b, b->stream, 0, b->streams, first, count, pool_offset, input, output,
                         rope);
}

/* Stream groups of the step: tiles of 16 streams dealt into `groups` runs.
 * Returns the group count actually used (a group holds >= 1 tile). */
static size_t group_bounds(const PhononFlowBatch *b, size_t *first, size_t *count) {
    const size_t tiles = (b->streams + 15) / 16;
    /* A prefill's attention work list spans all its pseudo-streams: one group. */
    const size_t want = b->pre.active ? 1 : b->groups;
    const size_t groups = want < tiles ? want : tiles;
    for (size_t g = 0; g < groups; g++) {
        const size_t t0 = tiles * g / groups, t1 = tiles * (g + 1) / groups;
        first[g] = t0 * 16;
        const size_t end = t1 * 16 < b->streams ? t1 * 16 : b->streams;
        count[g] = end - first[g];
    }
    return groups;
}

/* One step: each stream group runs all layers on its own HIP stream (forked
 * from and joined back into the batch stream), so one group's latency-bound
 * projections overlap another group's bandwidth-bound attention. */
static int enqueue_step(PhononFlowBatch *b, const float *input, float *output, float theta) {
    const float *rope = ph_rope_table(theta);
    size_t first[PH_MAX_GROUPS], count[PH_MAX_GROUPS];
    const size_t groups = group_bounds(b, first, count);
    if (!rope || !groups)
        return 0;
    if (groups > 1 && !pgpu_event_record(b->fork, b->stream))
        return 0;
    for (size_t g = 1; g < groups; g++)
        if (!pgpu_stream_wait_event(b->side[g - 1], b->fork))
            return 0;
    for (size_t g = 0; g < groups; g++)
        if (!enqueue_group(b, g ? b->side[g - 1] : b->stream, first[g], count[g], 0,
                           b->model->layers, 0, input, output, rope))
            return 0;
    for (size_t g = 1; g < groups; g++)
        if (!pgpu_event_record(b->join[g - 1], b->side[g - 1]) ||
            !pgpu_stream_wait_event(b->stream, b->join[g - 1]))
            return 0;
    return pgpu_advance_positions(b->stream, b->positions, (int)b->streams, 1);
}

/* ------------------------------------------------------ one-launch step -- */

/* Floats of one (layer, stream, head) group of (max, sum) pairs: padded to
 * whole 128-byte lines, so no two groups share a cache line. */
static size_t flow_ml_group(const PhononFlowBatch *b) {
    return (2 * b->max_splits + 31) / 32 * 32;
}

/* When a step runs as one launch: always (flow = 2), or, by default
 * (flow = 1), for the decode batch sizes where it measured faster on MI355X
 * than one launch per phase (PH_FLOW_MIN_TILES..PH_FLOW_MAX_TILES 16-stream
 * tiles; prefill and larger batches are attention-bound, where the separate
 * attention kernel streams K/V faster). */
/* Splits per ATTN task: one for a few streams (the step is a latency
 * chain) and at 3 and 4 tiles, two otherwise (fewer, longer attention tasks
 * keep more K/V in flight per work-group slot); measured on MI355X. */
static int flow_rounds(const PhononFlowBatch *b) {
    if (b->fl.rounds_set)
        return b->fl.rounds_set;
    const size_t tiles = (b->streams + 15) / 16;
    return b->streams <= PH_FLOW_ONE_ROUND_MAX_STREAMS ||
                   (tiles >= PH_FLOW_ONE_ROUND_MIN_TILES && tiles <= PH_FLOW_ONE_ROUND_MAX_TILES)
               ? 1
               : PGPU_FLOW_ATTN_ROUNDS;
}

static int flow_usable(const PhononFlowBatch *b, int prefill) {
    if (!b->flow || b->model->q8 < 0 || b->model->layers > 63 || b->streams > 4096)
        return 0;
    const size_t tiles = (b->streams + 15) / 16;
    return b->flow == 2 ||
           (!prefill && tiles >= PH_FLOW_MIN_TILES && tiles <= PH_FLOW_MAX_TILES);
}

/* Every tagged hand-off word to tag 0 and the next step's tag to 1: no
 * stale word carries a tag a later step uses until the tag wraps. */
static int flow_clear_tags(PhononFlowBatch *b) {
    b->fl.tag = 1;
    return pgpu_memset(b->stream, b->fl.rows, 0, b->fl.rows_words * sizeof(uint64_t)) &&
           pgpu_memset(b->stream, b->fl.parts, 0, b->fl.parts_words * sizeof(uint64_t));
}

/* Grows the per-layer buffers of the one-launch step to hold `streams`
 * streams of the model's layers. Every value a step's task hands to another
 * has its own address per layer (see pgpu_flow.hip). */
static int flow_reserve(PhononFlowBatch *b, size_t streams) {
    const size_t cap = (streams + 15) / 16 * 16, layers = b->model->layers;
    if (cap <= b->fl.cap && layers <= b->fl.cap_layers)
        return 1;
    const size_t new_cap = cap > b->fl.cap ? cap : b->fl.cap;
    const size_t new_layers = layers > b->fl.cap_layers ? layers : b->fl.cap_layers;
    if (!pgpu_stream_sync(b->stream))
        return 0;
    drop_graphs(b);
    void *old[] = {b->fl.act,      b->fl.part_acc, b->fl.part_ml, b->fl.hidden,
                   b->fl.counters, b->fl.rows,     b->fl.parts,   b->fl.mlp_parts};
    for (size_t i = 0; i < sizeof(old) / sizeof(old[0]); i++)
        pgpu_free(old[i]);
    b->fl.act = NULL;
    b->fl.part_acc = b->fl.part_ml = NULL;
    b->fl.hidden = NULL;
    b->fl.counters = NULL;
    b->fl.rows = b->fl.parts = NULL;
    b->fl.mlp_parts = NULL;
    b->fl.mlp_words = 0;
    b->fl.cap = b->fl.cap_layers = 0;
    b->fl.streams = 0; /* the schedule is rebuilt against the new buffers */
    const size_t groups = new_layers * new_cap * PH_HEADS;
    /* a multiple of 64 words: each set starts on a 256-byte line */
    b->fl.counter_words =
        (new_layers * (new_cap / 16) * PGPU_FLOW_KINDS * PGPU_FLOW_COUNTER_STRIDE + groups + 63) /
        64 * 64;
    b->fl.act = pgpu_malloc(new_layers * 4 * new_cap * PH_WIDTH * sizeof(float));
    b->fl.part_acc = pgpu_malloc(groups * b->max_splits * 64 * sizeof(float));
    b->fl.part_ml = pgpu_malloc(groups * flow_ml_group(b) * sizeof(float));
    b->fl.hidden = pgpu_malloc(new_layers * new_cap * PH_FFN * 3 * sizeof(uint16_t));
    b->fl.counters = pgpu_malloc(2 * b->fl.counter_words * sizeof(unsigned));
    b->fl.rows_words = new_layers * 6 * new_cap * PH_WIDTH;
    b->fl.parts_words = groups * b->max_splits * PGPU_FLOW_PART_WORDS;
    b->fl.rows = pgpu_malloc(b->fl.rows_words * sizeof(uint64_t));
    b->fl.parts = pgpu_malloc(b->fl.parts_words * sizeof(uint64_t));
    b->fl.parity = 0;
    if (!b->fl.act || !b->fl.part_acc || !b->fl.part_ml || !b->fl.hidden || !b->fl.counters ||
        !b->fl.rows || !b->fl.parts ||
        !pgpu_memset(b->stream, b->fl.counters, 0, 2 * b->fl.counter_words * sizeof(unsigned)) ||
        !pgpu_memset(b->stream, b->fl.hidden, 0,
                     new_layers * new_cap * PH_FFN * 3 * sizeof(uint16_t)) ||
        !flow_clear_tags(b) || !pgpu_stream_sync(b->stream))
        return 0;
    b->fl.cap = new_cap;
    b->fl.cap_layers = new_layers;
    return 1;
}

/* How a one-launch step hands values between its tasks (pgpu_flow.hip).
 * Tagged words save one memory round trip per hand-off, but every poll
 * fetches from memory, which costs more than the counter mode's shared
 * loads once the tile holds more than a few streams (measured on MI355X,
 * us per 12-layer step, contexts U{1..2048}, counter vs tagged: B = 1: 324
 * vs 291; B = 16: 482 vs 529). For those few streams, the out projection
 * merges the split partials itself, which removes the merging attention
 * task's hop (tagged vs merged in the out projection: B = 1: 319 vs 300;
 * B = 2: 329 vs 315; B = 3: 327 vs 319; B = 4: 343 vs 342). Up to two
 * streams, the fused MLP also removes the MLP-out hop; with more, its
 * QKV tasks' per-stream partial sums cost more than the hop (merge in the
 * out projection vs fused MLP, contexts U{1..2048}: B = 1: 276 vs 256;
 * B = 2: 300 vs 285; B = 3: 307 vs 314; B = 4: 330 vs 354). */
static int flow_tagged(const PhononFlowBatch *b) {
    if (b->fl.tagged_set >= 0)
        return b->fl.tagged_set;
    if (b->streams <= PH_FLOW_FUSED_DEFAULT_MAX_STREAMS)
        return PGPU_FLOW_HANDOFF_FUSED_MLP;
    return b->streams <= PH_FLOW_TAGGED_MAX_STREAMS ? PGPU_FLOW_HANDOFF_MERGE_OUT
                                                    : PGPU_FLOW_HANDOFF_COUNTER;
}

/* The hand-off mode a step runs in: the fused MLP only for a decode step of
 * at most PGPU_FLOW_FUSED_MAX_STREAMS streams (otherwise the merge in the
 * out projection, whose hand-offs it extends). */
static int flow_mode(const PhononFlowBatch *b, int prefill) {
    const int mode = flow_tagged(b);
    if (mode == PGPU_FLOW_HANDOFF_FUSED_MLP &&
        (prefill || b->streams > PGPU_FLOW_FUSED_MAX_STREAMS))
        return PGPU_FLOW_HANDOFF_MERGE_OUT;
    return mode;
}

/* Rebuilds (and uploads) the step's task list (pgpu_flow_schedule) when the
 * streams, the layers or a context outgrow it. A stream lists the splits of
 * its context PH_FLOW_HEADROOM positions ahead; tasks past its live context
 * end at once. */
static int flow_schedule(PhononFlowBatch *b, int prefill) {
    const size_t streams = b->streams, layers = b->model->layers;
    const int rounds = flow_rounds(b);
    const int fused = flow_mode(b, prefill) == PGPU_FLOW_HANDOFF_FUSED_MLP;
    const int flags = (prefill ? PGPU_FLOW_SCHEDULE_PREFILL : 0) |
                      (fused ? PGPU_FLOW_SCHEDULE_FUSED_MLP : 0);
    int valid = b->fl.streams == streams && b->fl.layers == layers && b->fl.prefill == prefill &&
                b->fl.rounds == rounds && b->fl.fused == fused;
    for (size_t s = 0; valid && s < streams; s++)
        valid = (b->host_positions[s] + PH_SPLIT_KEYS) / PH_SPLIT_KEYS <= b->fl.cover[s];
    if (valid)
        return 1;
    b->fl.streams = 0; /* no valid schedule until the new one is uploaded */
    for (size_t s = 0; s < streams; s++) {
        size_t need = (b->host_positions[s] + PH_FLOW_HEADROOM + PH_SPLIT_KEYS) / PH_SPLIT_KEYS;
        b->fl.cover[s] = need < b->max_splits ? need : b->max_splits;
        b->fl.units[s] = (b->fl.cover[s] + rounds - 1) / rounds;
    }
    const pgpu_flow_placement place =
        b->fl.place_set ? b->fl.place : ph_flow_default_placement(rounds);
    const size_t tasks =
        pgpu_flow_schedule(streams, layers, b->fl.units, &place, flags, NULL, 0);
    if (tasks > b->fl.host_cap) {
        uint32_t *grown = realloc(b->fl.host_schedule, tasks * sizeof(uint32_t));
        if (!grown)
            return 0;
        b->fl.host_schedule = grown;
        b->fl.host_cap = tasks;
    }
    uint32_t *d = b->fl.host_schedule;
    const size_t k = pgpu_flow_schedule(streams, layers, b->fl.units, &place, flags, d,
                                        b->fl.host_cap);
    if (k != tasks)
        return ph_fail("flow schedule: task count mismatch");
    if (!pgpu_stream_sync(b->stream))
        return 0;
    drop_graphs(b);
    if (tasks > b->fl.schedule_cap) {
        pgpu_free(b->fl.schedule);
        b->fl.schedule = pgpu_malloc(tasks * sizeof(uint32_t));
        b->fl.schedule_cap = b->fl.schedule ? tasks : 0;
        if (!b->fl.schedule)
            return 0;
    }
    if (!pgpu_copy_h2d(b->stream, b->fl.schedule, d, tasks * sizeof(uint32_t)))
        return 0;
    b->fl.rounds = rounds;
    b->fl.tasks = tasks;
    b->fl.streams = streams;
    b->fl.layers = layers;
    b->fl.prefill = prefill;
    b->fl.fused = fused;
    b->fl.version++;
    return 1;
}

/* Makes buffers and schedule ready for the batch's current streams (outside
 * any graph capture); called once per one-launch step. The tagged mode's
 * tag advances once per step: before it could come back to a value a stale
 * word still carries, every word is cleared. */
static int flow_prepare(PhononFlowBatch *b, int prefill) {
    if (!flow_reserve(b, b->streams) || !flow_schedule(b, prefill))
        return 0;
    if (b->fl.fused && !b->fl.mlp_parts) {
        /* [layers][MLP_IN tasks][16][512] fp32, read only after their count */
        const size_t words = b->fl.cap_layers * PGPU_FLOW_MLP_IN_TASKS * 16 * PH_WIDTH;
        b->fl.mlp_parts = pgpu_malloc(words * sizeof(float));
        if (!b->fl.mlp_parts)
            return 0;
        b->fl.mlp_words = words;
    }
    if (b->fl.tag >= UINT32_MAX - 1 && !(pgpu_stream_sync(b->stream) && flow_clear_tags(b)))
        return 0;
    return 1;
}


/* One step as a single launch. It uses one set of counters and zeroes the
 * other for the next step, and reads the positions as stored plus pos_lag
 * (the steps since they were last written), so that nothing has to run
 * between two steps. */
static int enqueue_flow(PhononFlowBatch *b, const float *input, float *output, float theta) {
    const PhononFlowModel *m = b->model;
    const float *rope = ph_rope_table(theta);
    const size_t tiles = (b->streams + 15) / 16, layers = m->layers;
    if (!rope)
        return 0;
    const size_t phase_words = layers * tiles * PGPU_FLOW_KINDS * PGPU_FLOW_COUNTER_STRIDE;
    const size_t used = (phase_words + layers * tiles * 16 * PH_HEADS + 3) / 4 * 4;
    unsigned *set = b->fl.counters + (size_t)b->fl.parity * b->fl.counter_words;
    unsigned *next = b->fl.counters + (size_t)(1 - b->fl.parity) * b->fl.counter_words;
    if (used > b->fl.counter_words ||
        (used + PGPU_FLOW_CLEAR_WORDS - 1) / PGPU_FLOW_CLEAR_WORDS > b->fl.tasks)
        return ph_fail("flow step: counters outgrow the clearing work-groups");
    const pgpu_flow_step f = {.layers = m->flow_layers,
                              .layer_count = (int)layers,
                              .q8 = m->q8,
                              .streams = (int)b->streams,
                              .tiles = (int)tiles,
                              .prefill = b->fl.prefill,
                              .pool_offset = 0,
                              .input = input,
                              .output = output,
                              .act = b->fl.act,
                              .hidden = b->fl.hidden,
                              .part_acc = b->fl.part_acc,
                              .part_ml = b->fl.part_ml,
                              .max_splits = (int)b->max_splits,
                              .ml_group = (int)flow_ml_group(b),
                              .tables = b->tables,
                              .positions = b->positions,
                              .pos_delta = b->pos_lag,
                              .table_stride = (int)b->table_len,
                              .rope = rope,
                              .schedule = b->fl.schedule,
                              .tasks = (unsigned)b->fl.tasks,
                              .phase = set,
                              .split_done = set + phase_words,
                              .clear = next,
                              .clear_words = (unsigned)used,
                              .status = b->status,
                              .trace = b->fl.trace_cap >= b->fl.tasks ? b->fl.trace : NULL,
                              .attn_rounds = b->fl.rounds,
                              .wait_us = b->fl.wait_us,
                              .tagged = flow_mode(b, b->fl.prefill),
                              .rows = b->fl.rows,
                              .parts = b->fl.parts,
                              .tag = b->fl.tag,
                              .mlp_parts = b->fl.mlp_parts};
    if (!((!b->time_before || pgpu_event_record(b->time_before, b->stream)) &&
          pgpu_flow_launch(b->stream, &f, &b->pool->kv) &&
          (!b->time_after || pgpu_event_record(b->time_after, b->stream))))
        return 0;
    b->fl.parity = 1 - b->fl.parity;
    b->fl.tag++;
    b->pos_lag++;
    return 1;
}

/* Work entries of the prefill attention (pgpu_prefill_attention): for each
 * stream i (pseudo-streams from its offset on) and each 256-key split j of
 * its context, its positions that reach split j, in runs of `run`
 * consecutive positions. Returns the entry count; writes them when `out`
 * holds that many. */
static size_t entry_list(size_t streams, const size_t *first, const size_t *counts, size_t run,
                         int32_t *out, size_t cap) {
    size_t n = 0, offset = 0;
    for (size_t i = 0; i < streams; i++) {
        const size_t last = first[i] + counts[i] - 1;
        for (size_t j = 0; j <= last / PH_SPLIT_KEYS; j++) {
            const size_t start = j * PH_SPLIT_KEYS;
            const size_t k0 = start > first[i] ? start - first[i] : 0;
            for (size_t k = k0; k < counts[i]; k += run, n++) {
                if (n < cap) {
                    const size_t k1 = k + run < counts[i] ? k + run : counts[i];
                    out[4 * n] = (int32_t)(offset + k);
                    out[4 * n + 1] = (int32_t)(offset + k1);
                    out[4 * n + 2] = (int32_t)j;
                    out[4 * n + 3] = 0;
                }
            }
        }
        offset += counts[i];
    }
    return n;
}

/* A prefill call's small uploads (block tables, positions, work lists) are
 * laid out in one pinned staging area whose device mirror has the same
 * layout: stage_put places a piece and returns its device address, and
 * stage_flush moves the whole area up as one asynchronous copy on the
 * batch's stream (one copy instead of one per piece, and no host round
 * trip). The kernels read the pieces where the copy puts them. stage_begin
 * runs after the stream was synchronized, so no copy or kernel of an
 * earlier call still reads either area. */
static int stage_begin(PhononFlowBatch *b, size_t bytes) {
    if (bytes > b->pre.stage_cap) {
        pgpu_host_free(b->pre.stage);
        pgpu_free(b->pre.stage_dev);
        b->pre.stage = pgpu_host_malloc(bytes);
        b->pre.stage_dev = pgpu_malloc(bytes);
        b->pre.stage_cap = b->pre.stage && b->pre.stage_dev ? bytes : 0;
        if (!b->pre.stage_cap)
            return 0;
    }
    b->pre.stage_used = 0;
    return 1;
}

static const int32_t *stage_put(PhononFlowBatch *b, const void *src, size_t bytes) {
    const size_t at = (b->pre.stage_used + 255) & ~(size_t)255;
    if (at > b->pre.stage_cap || bytes > b->pre.stage_cap - at) {
        ph_fail("prefill: staging area too small");
        return NULL;
    }
    memcpy(b->pre.stage + at, src, bytes);
    b->pre.stage_used = at + bytes;
    return (const int32_t *)(b->pre.stage_dev + at);
}

static int stage_flush(PhononFlowBatch *b) {
    return pgpu_copy_h2d_async(b->stream, b->pre.stage_dev, b->pre.stage, b->pre.stage_used);
}

/* Staging bytes of a prefill of `total` positions: positions and table map,
 * the three attention work lists at their 65535-entry limits, and `extra`. */
static size_t stage_bytes(size_t total, size_t extra) {
    return extra + 2 * total * sizeof(int32_t) + 65535 * (4 + 2 + 4) * sizeof(int32_t) +
           8 * 256;
}

/* The prefill attention's work list, uploaded: positions per entry halved
 * from PH_PREFILL_RUN while the list would give fewer than
 * PH_PREFILL_MIN_GROUPS work-groups (8 per entry), so a short prompt still
 * spreads over the GPU. */
static int prefill_entries(PhononFlowBatch *b, size_t streams, const size_t *first,
                           const size_t *counts) {
    size_t run = PH_PREFILL_RUN;
    size_t n = entry_list(streams, first, counts, run, NULL, 0);
    while (run > 8 && n * PH_HEADS < PH_PREFILL_MIN_GROUPS) {
        run /= 2;
        n = entry_list(streams, first, counts, run, NULL, 0);
    }
    if (!n || n > 65535)
        return ph_fail("prefill: attention work list size out of range");
    if (n > b->pre.cap) {
        int32_t *host = realloc(b->pre.host, n * 4 * sizeof(int32_t));
        if (!host)
            return 0;
        b->pre.host = host;
        b->pre.cap = n;
    }
    if (entry_list(streams, first, counts, run, b->pre.host, b->pre.cap) != n)
        return 0;
    b->pre.count = n;
    return (b->pre.entries = stage_put(b, b->pre.host, n * 4 * sizeof(int32_t))) != NULL;
}

/* Work list of the run-based prefill attentions (pgpu_prefill_attention_mfma
 * and _rows):
 * runs of up to 64 consecutive positions of one stream, as (first
 * pseudo-stream, count), the runs with the most keys first so that the
 * longest work-groups start earliest. */
typedef struct {
    size_t last;
    int32_t s0, n;
} PrefillRun;

static int run_order(const void *x, const void *y) {
    const PrefillRun *a = x, *b = y;
    return a->last < b->last ? 1 : (a->last > b->last ? -1 : (a->s0 > b->s0) - (a->s0 < b->s0));
}

/* Work list of pgpu_prefill_attention_mfma: a stream's runs paired so that
 * its run with the most keys shares a work-group with the one with the
 * fewest (the causal mask makes a run's work grow with its last position),
 * then the pairs with the most keys first. A stream with an odd number of
 * runs leaves its middle run unpaired. */
typedef struct {
    size_t keys;
    int32_t s0, n, s1, n1;
} PrefillPair;

static int pair_order(const void *x, const void *y) {
    const PrefillPair *a = x, *b = y;
    return a->keys < b->keys ? 1 : (a->keys > b->keys ? -1 : (a->s0 > b->s0) - (a->s0 < b->s0));
}

/* Runs of a short prompt (at most 512 positions in the call): 16 positions,
 * so that its attention spreads over more work-groups (the B=1 workload's
 * 256-position prefill: 0.692 ms with runs of 64, 0.679 with 32, 0.674
 * with 16; a run's work-group still streams its keys once). */
enum { PH_PREFILL_SHORT_RUN = 16 };

static int prefill_pairs(PhononFlowBatch *b, size_t streams, const size_t *first,
                         const size_t *counts) {
    size_t n = 0, total = 0;
    for (size_t i = 0; i < streams; i++)
        total += counts[i];
    const size_t run = total <= 512 ? PH_PREFILL_SHORT_RUN : PH_PREFILL_RUN;
    for (size_t i = 0; i < streams; i++)
        n += ((counts[i] + run - 1) / run + 1) / 2;
    PrefillPair *list = malloc(n * sizeof(PrefillPair));
    if (!list)
        return 0;
    size_t k = 0;
    for (size_t i = 0, offset = 0; i < streams; offset += counts[i], i++) {
        const size_t runs = (counts[i] + run - 1) / run; /* >= 1 */
        for (size_t lo = 0, hi = runs - 1;; lo++, hi--) {
            /* Run j: positions [run j, min(run (j + 1), count)) of the stream;
             * a run paired as `lo` is never the stream's last, so it is full. */
            const size_t q_hi = hi * run, q_lo = lo * run;
            const size_t n_hi = counts[i] - q_hi < run ? counts[i] - q_hi : run;
            list[k] = (PrefillPair){first[i] + q_hi + n_hi, (int32_t)(offset + q_hi),
                                    (int32_t)n_hi, 0, 0};
            if (lo < hi) {
                list[k].s1 = (int32_t)(offset + q_lo);
                list[k].n1 = (int32_t)run;
                list[k].keys += first[i] + q_lo + run;
            }
            k++;
            if (lo + 1 >= hi)
                break;
        }
    }
    n = k;
    qsort(list, n, sizeof(PrefillPair), pair_order);
    if (n > b->pre.pairs_cap) {
        int32_t *host = realloc(b->pre.pairs_host, n * 4 * sizeof(int32_t));
        if (!host) {
            free(list);
            return 0;
        }
        b->pre.pairs_host = host;
        b->pre.pairs_cap = n;
    }
    for (size_t j = 0; j < n; j++) {
        b->pre.pairs_host[4 * j] = list[j].s0;
        b->pre.pairs_host[4 * j + 1] = list[j].n;
        b->pre.pairs_host[4 * j + 2] = list[j].s1;
        b->pre.pairs_host[4 * j + 3] = list[j].n1;
    }
    free(list);
    b->pre.pairs_count = n;
    return (b->pre.pairs = stage_put(b, b->pre.pairs_host, n * 4 * sizeof(int32_t))) != NULL;
}

static int prefill_runs(PhononFlowBatch *b, size_t streams, const size_t *first,
                        const size_t *counts) {
    size_t n = 0;
    for (size_t i = 0; i < streams; i++)
        n += (counts[i] + PH_PREFILL_RUN - 1) / PH_PREFILL_RUN;
    if (!n || n > 65535)
        return ph_fail("prefill: attention work list size out of range");
    PrefillRun *list = malloc(n * sizeof(PrefillRun));
    if (!list)
        return 0;
    for (size_t i = 0, k = 0, offset = 0; i < streams; offset += counts[i], i++)
        for (size_t q = 0; q < counts[i]; q += PH_PREFILL_RUN, k++) {
            const size_t len = counts[i] - q < PH_PREFILL_RUN ? counts[i] - q : PH_PREFILL_RUN;
            list[k] = (PrefillRun){first[i] + q + len - 1, (int32_t)(offset + q), (int32_t)len};
        }
    qsort(list, n, sizeof(PrefillRun), run_order);
    if (n > b->pre.runs_cap) {
        int32_t *host = realloc(b->pre.runs_host, n * 2 * sizeof(int32_t));
        if (!host) {
            free(list);
            return 0;
        }
        b->pre.runs_host = host;
        b->pre.runs_cap = n;
    }
    for (size_t k = 0; k < n; k++) {
        b->pre.runs_host[2 * k] = list[k].s0;
        b->pre.runs_host[2 * k + 1] = list[k].n;
    }
    free(list);
    b->pre.runs_count = n;
    return (b->pre.runs = stage_put(b, b->pre.runs_host, n * 2 * sizeof(int32_t))) != NULL &&
           prefill_pairs(b, streams, first, counts);
}

/* Pseudo-streams of a batched prefill: position first[i] + k (k < counts[i])
 * of stream i becomes its own stream with block-table row i of tables_dev
 * (device, [streams][table_len]). A step then runs every such position
 * through all layers at once: each layer's projection appends the K/V of all
 * of them before its attention runs, and position p attends p + 1 keys, so
 * the pass is causal and computes what `counts` consecutive steps would. */
static size_t prefill_total(const PhononFlowBatch *b, size_t streams, const size_t *first,
                            const size_t *counts) {
    size_t total = 0;
    for (size_t i = 0; i < streams; i++) {
        if (!counts[i] || first[i] >= b->max_positions ||
            counts[i] > b->max_positions - first[i] || counts[i] > b->max_streams - total)
            return 0;
        total += counts[i];
    }
    return total;
}

/* ph_batch_set_prefill after the stream was synchronized and the staging
 * area begun (it holds stage_bytes(total, 0) more). */
static int set_prefill(PhononFlowBatch *b, size_t streams, const size_t *first,
                       const size_t *counts, const int32_t *tables_dev) {
    const size_t total = prefill_total(b, streams, first, counts);
    if (!total)
        return 0;
    if (!b->pre.split &&
        !(b->pre.split = pgpu_malloc(b->padded_streams / 16 * (PH_WIDTH / 32) * 1536 *
                                     sizeof(uint16_t))))
        return 0;
    int32_t *pos32 = malloc(total * sizeof(int32_t)), *map = malloc(total * sizeof(int32_t));
    int ok = pos32 && map;
    for (size_t i = 0, p = 0; ok && i < streams; i++)
        for (size_t k = 0; k < counts[i]; k++, p++) {
            pos32[p] = (int32_t)(first[i] + k);
            map[p] = (int32_t)i;
            b->host_positions[p] = first[i] + k;
        }
    const int32_t *pos_dev = NULL;
    ok = ok && (pos_dev = stage_put(b, pos32, total * sizeof(int32_t))) &&
         (b->table_map = stage_put(b, map, total * sizeof(int32_t))) &&
         prefill_entries(b, streams, first, counts) && prefill_runs(b, streams, first, counts) &&
         stage_flush(b) &&
         pgpu_gather_rows_copy(b->stream, b->tables, tables_dev, b->table_map, (int)total,
                               (int)b->table_len, b->positions, pos_dev);
    free(pos32);
    free(map);
    if (ok) {
        b->streams = total;
        b->pos_lag = 0;
        b->pre.active = 1;
    }
    return ok;
}

int ph_batch_set_prefill(PhononFlowBatch *b, size_t streams, const size_t *first,
                         const size_t *counts, const int32_t *tables_dev) {
    const size_t total = prefill_total(b, streams, first, counts);
    return total && pgpu_stream_sync(b->stream) && stage_begin(b, stage_bytes(total, 0)) &&
           set_prefill(b, streams, first, counts, tables_dev);
}

int phonon_flow_batch_prefill_device(PhononFlowBatch *b, size_t streams, const size_t *first,
                                     const size_t *counts, const int32_t *tables,
                                     size_t table_len, const float *inputs, float theta,
                                     float *outputs) {
    if (!b || !streams || streams > b->max_streams || !first || !counts || !tables ||
        table_len != b->table_len || !inputs || !outputs || !isfinite(theta) || theta <= 0.0f)
        return 0;
    const size_t total = prefill_total(b, streams, first, counts),
                 table_bytes = streams * table_len * sizeof(int32_t);
    if (!total || !pgpu_stream_sync(b->stream) ||
        !stage_begin(b, stage_bytes(total, table_bytes)) ||
        !(b->table_src = stage_put(b, tables, table_bytes)) ||
        !set_prefill(b, streams, first, counts, b->table_src))
        return 0;
    if (flow_usable(b, 1))
        return flow_prepare(b, 1) && enqueue_flow(b, inputs, outputs, theta);
    return (b->splits = splits_for(b, 0)) > 0 && enqueue_step(b, inputs, outputs, theta);
}

int phonon_flow_batch_set_wait_limit(PhononFlowBatch *b, unsigned microseconds) {
    if (!b || microseconds > 10000000u)
        return 0;
    b->fl.wait_us = microseconds;
    return 1;
}

int phonon_flow_batch_set_prefill_exact(PhononFlowBatch *b, int exact) {
    if (!b || exact < 0 || exact > 2)
        return 0;
    b->pre.exact = exact;
    return 1;
}

int phonon_flow_batch_set_groups(PhononFlowBatch *b, size_t groups) {
    if (!b || !groups || groups > PH_MAX_GROUPS)
        return 0;
    if (groups > 1) {
        /* each made once; a failure leaves the groups as they were */
        int ok = b->fork || pgpu_event_create(&b->fork);
        for (size_t g = 0; ok && g + 1 < PH_MAX_GROUPS; g++)
            ok = (b->side[g] || pgpu_stream_create(&b->side[g])) &&
                 (b->join[g] || pgpu_event_create(&b->join[g]));
        if (!ok)
            return 0;
    }
    if (b->groups != groups) {
        drop_graphs(b);
        b->groups = groups;
    }
    return 1;
}

int phonon_flow_batch_set_placement(PhononFlowBatch *b, const pgpu_flow_placement *place) {
    if (!b)
        return 0;
    b->fl.place = place ? *place : ph_flow_default_placement(1);
    b->fl.place_set = place != NULL;
    b->fl.streams = 0; /* rebuild the task list */
    drop_graphs(b);
    return 1;
}

int phonon_flow_batch_set_trace(PhononFlowBatch *b, uint64_t *trace, size_t capacity) {
    if (!b || (!trace) != (!capacity))
        return 0;
    drop_graphs(b);
    b->fl.trace = trace;
    b->fl.trace_cap = capacity;
    return 1;
}

size_t phonon_flow_batch_schedule(const PhononFlowBatch *b, uint32_t *schedule,
                                  size_t capacity) {
    if (!b || !b->fl.streams)
        return 0;
    if (schedule && capacity >= b->fl.tasks)
        memcpy(schedule, b->fl.host_schedule, b->fl.tasks * sizeof(uint32_t));
    return b->fl.tasks;
}

int phonon_flow_batch_set_pipeline(PhononFlowBatch *b, int mode) {
    if (!b || mode < 0 || mode > 2)
        return 0;
    if (b->flow != mode) {
        drop_graphs(b);
        b->flow = mode;
    }
    return 1;
}

int phonon_flow_batch_set_handoff(PhononFlowBatch *b, int tagged) {
    if (!b || tagged < -1 || tagged > PGPU_FLOW_HANDOFF_FUSED_MLP)
        return 0;
    b->fl.tagged_set = tagged;
    return 1;
}

int phonon_flow_batch_set_attention_rounds(PhononFlowBatch *b, int rounds) {
    if (!b || rounds < 0 || rounds > PGPU_FLOW_ATTN_ROUNDS)
        return 0;
    b->fl.rounds_set = rounds;
    return 1;
}

int phonon_flow_batch_set_timing(PhononFlowBatch *b, void *before, void *after) {
    if (!b || (!before) != (!after))
        return 0;
    b->time_before = before;
    b->time_after = after;
    return 1;
}

int phonon_flow_batch_set_graph(PhononFlowBatch *b, int use_graph) {
    if (!b)
        return 0;
    b->eager = !use_graph;
    drop_graphs(b);
    return 1;
}

int phonon_flow_batch_step_device(PhononFlowBatch *b, const float *inputs, float theta,
                                  float *outputs) {
    if (!b || !b->streams || !inputs || !outputs)
        return 0;
    for (size_t s = 0; s < b->streams; s++)
        if (b->host_positions[s] >= b->max_positions)
            return 0;
    const int flow = flow_usable(b, 0);
    /* A one-launch step reads the positions as stored plus pos_lag; the
     * phase kernels (and a captured graph of them) read them as stored. */
    if (flow ? !flow_prepare(b, 0) : !fold_positions(b))
        return 0;
    /* A one-launch step is one kernel, launched directly (a graph launch
     * costs 7 us per step more on MI355X), with the step's tag, counter set
     * and position lag as arguments: it is never captured. */
    if (b->eager || b->time_before || flow) {
        b->splits = splits_for(b, 0);
        if (!(flow ? enqueue_flow(b, inputs, outputs, theta)
                   : enqueue_step(b, inputs, outputs, theta)))
            return 0;
        for (size_t s = 0; s < b->streams; s++)
            b->host_positions[s]++;
        return 1;
    }
    /* A captured phase-by-phase step covers contexts up to its attention
     * grid: captured with 256 positions of headroom, re-captured when a
     * context outgrows it. */
    const size_t need = splits_for(b, 0);
    void *exec = NULL;
    for (size_t i = 0; i < 2 && !exec; i++)
        if (b->graphs[i].exec && b->graphs[i].streams == b->streams &&
            b->graphs[i].splits >= need && b->graphs[i].theta == theta &&
            b->graphs[i].input == inputs && b->graphs[i].output == outputs)
            exec = b->graphs[i].exec;
    if (!exec) {
        const size_t slot = b->graph_victim;
        pgpu_graph_destroy(b->graphs[slot].exec);
        b->graphs[slot].exec = NULL;
        b->splits = splits_for(b, PH_SPLIT_KEYS);
        if (!ph_rope_table(theta) || !pgpu_graph_begin(b->stream))
            return 0;
        const int enqueued = enqueue_step(b, inputs, outputs, theta);
        const int ended = pgpu_graph_end(b->stream, &exec);
        if (!enqueued || !ended) {
            pgpu_graph_destroy(exec);
            return 0;
        }
        b->graphs[slot].exec = exec;
        b->graphs[slot].streams = b->streams;
        b->graphs[slot].splits = b->splits;
        b->graphs[slot].theta = theta;
        b->graphs[slot].input = inputs;
        b->graphs[slot].output = outputs;
        b->graph_victim = 1 - slot;
    }
    if (!pgpu_graph_launch(exec, b->stream))
        return 0;
    for (size_t s = 0; s < b->streams; s++)
        b->host_positions[s]++;
    return 1;
}

int phonon_flow_batch_status(PhononFlowBatch *b, int *status) {
    if (!b || !status || !pgpu_stream_sync(b->stream))
        return 0;
    return pgpu_copy_d2h(b->stream, status, b->status, sizeof(int));
}

int phonon_flow_batch_sync(PhononFlowBatch *b) {
    if (!b || !pgpu_stream_sync(b->stream))
        return 0;
    int st = 0;
    if (!pgpu_copy_d2h(b->stream, &st, b->status, sizeof(int)))
        return 0;
    if (st && !pgpu_memset(b->stream, b->status, 0, sizeof(int)))
        return 0;
    return pgpu_stream_sync(b->stream) && st == 0;
}

int phonon_flow_batch_step(PhononFlowBatch *b, const float *inputs, float theta,
                           float *outputs) {
    if (!b || !b->streams || !inputs || !outputs)
        return 0;
    const size_t bytes = b->streams * PH_WIDTH * sizeof(float);
    if (!pgpu_copy_h2d(b->stream, b->in, inputs, bytes) ||
        !phonon_flow_batch_step_device(b, b->in, theta, b->out))
        return 0;
    const int clean = phonon_flow_batch_sync(b);
    if (!pgpu_copy_d2h(b->stream, outputs, b->out, bytes))
        return 0;
    return clean && ph_all_finite(outputs, b->streams * PH_WIDTH);
}

int phonon_flow_batch_positions(const PhononFlowBatch *b, size_t *positions) {
    if (!b || !positions)
        return 0;
    memcpy(positions, b->host_positions, b->streams * sizeof(size_t));
    return 1;
}

void *phonon_flow_batch_stream(const PhononFlowBatch *b) { return b ? b->stream : NULL; }
float *phonon_flow_batch_device_inputs(PhononFlowBatch *b) { return b ? b->in : NULL; }
float *phonon_flow_batch_device_outputs(PhononFlowBatch *b) { return b ? b->out : NULL; }

int ph_batch_status(PhononFlowBatch *b) { return phonon_flow_batch_sync(b); }
float *ph_batch_in(PhononFlowBatch *b) { return b->in; }
float *ph_batch_out(PhononFlowBatch *b) { return b->out; }
size_t ph_batch_table_len(const PhononFlowBatch *b) { return b->table_len; }
const int32_t *ph_batch_tables(const PhononFlowBatch *b) { return b->tables; }
float *ph_batch_scratch_rows(PhononFlowBatch *b) { return b->rows; }
void *ph_batch_stream(const PhononFlowBatch *b) { return b->stream; }
int *ph_batch_status_word(PhononFlowBatch *b) { return b->status; }

/* ------------------------------------------------------------- registry -- */

typedef struct Registered {
    const PhononFlowLayerWeights *weights;
    size_t layers;
    const PhononTensorView *views[64][8];
    PhononFlowModel *model;
    struct Registered *next;
} Registered;

static pthread_mutex_t g_registry_lock = PTHREAD_MUTEX_INITIALIZER;
static Registered *g_registry;

static void snapshot_views(const PhononFlowLayerWeights *w, size_t layers,
                           const PhononTensorView *views[64][8]) {
    for (size_t l = 0; l < layers; l++) {
        const PhononTensorView *v[8] = {w[l].qkv,          w[l].attention_out, w[l].mlp_in,
                                        w[l].mlp_out,      w[l].norm1_weight,  w[l].norm1_bias,
                                        w[l].norm2_weight, w[l].norm2_bias};
        memcpy(views[l], v, sizeof(v));
    }
}

int phonon_flow_prepare_weights(const PhononFlowLayerWeights *weights, size_t layers) {
    if (!weights || !layers || layers > 64)
        return 0;
    Registered *r = calloc(1, sizeof(*r));
    if (!r || !phonon_flow_model_create(weights, layers, &r->model)) {
        free(r);
        return 0;
    }
    r->weights = weights;
    r->layers = layers;
    snapshot_views(weights, layers, r->views);
    phonon_flow_release_weights(weights);
    pthread_mutex_lock(&g_registry_lock);
    r->next = g_registry;
    g_registry = r;
    pthread_mutex_unlock(&g_registry_lock);
    return 1;
}

void phonon_flow_release_weights(const PhononFlowLayerWeights *weights) {
    pthread_mutex_lock(&g_registry_lock);
    for (Registered **p = &g_registry; *p;) {
        if ((*p)->weights == weights) {
            Registered *dead = *p;
            *p = dead->next;
            phonon_flow_model_destroy(dead->model);
            free(dead);
        } else {
            p = &(*p)->next;
        }
    }
    pthread_mutex_unlock(&g_registry_lock);
}

const PhononFlowModel *ph_registered_model(const PhononFlowLayerWeights *weights,
                                           size_t layers) {
    const PhononFlowModel *found = NULL;
    pthread_mutex_lock(&g_registry_lock);
    for (Registered *r = g_registry; r && !found; r = r->next) {
        if (r->weights != weights || r->layers != layers)
            continue;
        const PhononTensorView *now[64][8];
        snapshot_views(weights, layers, now);
        if (!memcmp(now, r->views, layers * sizeof(now[0])))
            found = r->model;
    }
    pthread_mutex_unlock(&g_registry_lock);
    return found;
}
