/* Drop-in single-stream decode step (phonon_transformer.h) on the MI355X.
 *
 * Each PhononKvCache keeps the reference's host arrays (tests and callers
 * read cache->keys directly) and gets a device copy: a paged pool with an
 * identity block table, found through the cache's `keys` pointer. Layers run
 * as a batch of one stream (phonon_flow_batch.c); the rows a step appends on
 * the device are copied back into keys/values before the call returns.
 * Weights come from phonon_flow_prepare_weights when registered, otherwise
 * they are uploaded for the call (and may change between calls).
 *
 * Concurrency (src/speech.h:40-41: requests on separate caches may run at
 * once): the library lock covers only finding the weights and the cache's
 * device copy; each copy has its own lock, batches and HIP stream, so steps
 * of different caches run at the same time on the host and the GPU. */
#include "ph_internal.h"

#include <limits.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct Mirror {
    const float *keys;
    size_t capacity, positions, table_len;
    PhononKvPool *pool;
    int32_t *table_host, *table_dev;
    PhononFlowBatch *batch;   /* one stream: decode steps */
    PhononFlowBatch *prefill; /* up to PH_PREFILL_CHUNK positions at once */
    pthread_mutex_t lock;     /* held by a step or prefill of this cache */
    struct Mirror *next;
} Mirror;

/* Positions a prefill runs through the layers together. */
enum { PH_PREFILL_CHUNK = 512 };

static Mirror *g_mirrors; /* guarded by ph_lock */

static void mirror_free(Mirror *m) {
    if (!m)
        return;
    phonon_flow_batch_destroy(m->batch);
    phonon_flow_batch_destroy(m->prefill);
    phonon_kv_pool_destroy(m->pool);
    free(m->table_host);
    if (m->table_dev) {
        (void)pgpu_stream_sync(ph_stream());
        pgpu_free(m->table_dev);
    }
    pthread_mutex_destroy(&m->lock);
    free(m);
}

static Mirror *mirror_find(const PhononKvCache *cache) {
    for (Mirror *m = g_mirrors; m; m = m->next)
        if (m->keys == cache->keys && m->capacity == cache->capacity)
            return m;
    return NULL;
}

static void mirror_drop(const float *keys) {
    for (Mirror **p = &g_mirrors; *p;) {
        if ((*p)->keys == keys) {
            Mirror *dead = *p;
            *p = dead->next;
            mirror_free(dead);
        } else {
            p = &(*p)->next;
        }
    }
}

/* Creates the device copy of a cache; rows [0, cache->length) of every layer
 * are uploaded from the host arrays. */
static Mirror *mirror_create(const PhononKvCache *cache) {
    if (!ph_init())
        return NULL;
    Mirror *m = calloc(1, sizeof(*m));
    if (!m)
        return NULL;
    if (pthread_mutex_init(&m->lock, NULL)) {
        free(m);
        return NULL;
    }
    m->keys = cache->keys;
    m->capacity = cache->capacity;
    m->positions = cache->capacity < PHONON_FLOW_MAX_POSITIONS ? cache->capacity
                                                               : PHONON_FLOW_MAX_POSITIONS;
    m->table_len = (m->positions + 15) / 16;
    int32_t *table = malloc(m->table_len * sizeof(int32_t));
    int ok = table && phonon_kv_pool_create(PHONON_FLOW_LAYERS, m->table_len, &m->pool) &&
             phonon_kv_pool_alloc(m->pool, m->table_len, table);
    if (ok) {
        m->table_dev = pgpu_malloc(m->table_len * sizeof(int32_t));
        ok = m->table_dev &&
             pgpu_copy_h2d(ph_stream(), m->table_dev, table, m->table_len * sizeof(int32_t));
    }
    const size_t rows = cache->length < m->positions ? cache->length : m->positions;
    if (ok && rows && cache->keys && cache->values)
        ok = phonon_kv_pool_write(m->pool, table, m->table_len, 0, rows, cache->keys,
                                  cache->values, cache->capacity);
    m->table_host = table;
    if (!ok) {
        mirror_free(m);
        return NULL;
    }
    m->next = g_mirrors;
    g_mirrors = m;
    return m;
}

static Mirror *mirror_get(const PhononKvCache *cache) {
    Mirror *m = mirror_find(cache);
    return m ? m : mirror_create(cache);
}

/* ------------------------------------------------------------- KV cache -- */

int phonon_kv_cache_init(PhononKvCache *cache, size_t capacity) {
    if (!cache || !capacity ||
        capacity > SIZE_MAX / (PHONON_FLOW_WIDTH * PHONON_FLOW_LAYERS * sizeof(float)))
        return 0;
    memset(cache, 0, sizeof(*cache));
    const size_t count = capacity * PHONON_FLOW_WIDTH * PHONON_FLOW_LAYERS;
    cache->keys = calloc(count, sizeof(float));
    cache->values = calloc(count, sizeof(float));
    if (!cache->keys || !cache->values) {
        phonon_kv_cache_destroy(cache);
        return 0;
    }
    cache->capacity = capacity;
    ph_lock();
    mirror_drop(cache->keys);
    Mirror *m = mirror_create(cache);
    ph_unlock();
    if (!m) {
        phonon_kv_cache_destroy(cache);
        return 0;
    }
    return 1;
}

void phonon_kv_cache_reset(PhononKvCache *cache) {
    if (cache)
        cache->length = 0;
}

void phonon_kv_cache_destroy(PhononKvCache *cache) {
    if (!cache)
        return;
    if (cache->keys) {
        ph_lock();
        mirror_drop(cache->keys);
        ph_unlock();
    }
    free(cache->keys);
    free(cache->values);
    memset(cache, 0, sizeof(*cache));
}

int phonon_kv_cache_append(PhononKvCache *cache, size_t layer, size_t position, const float *key,
                           const float *value, size_t width) {
    if (!cache || !cache->keys || !cache->values || !key || !value || width != PHONON_FLOW_WIDTH ||
        layer >= PHONON_FLOW_LAYERS || position >= cache->capacity)
        return 0;
    if (!ph_all_finite(key, width) || !ph_all_finite(value, width))
        return 0;
    const size_t offset = (layer * cache->capacity + position) * width;
    memcpy(cache->keys + offset, key, width * sizeof(float));
    memcpy(cache->values + offset, value, width * sizeof(float));
    ph_lock();
    Mirror *m = mirror_get(cache);
    int ok = m != NULL;
    if (ok && position < m->positions) {
        float *rows = ph_scratch(0, 2 * width * sizeof(float));
        int *status = ph_scratch(1, sizeof(int));
        int st = 0;
        void *s = ph_stream();
        ok = rows && status && pgpu_memset(s, status, 0, sizeof(int)) &&
             pgpu_copy_h2d(s, rows, key, width * sizeof(float)) &&
             pgpu_copy_h2d(s, rows + width, value, width * sizeof(float)) &&
             pgpu_kv_copy(s, ph_pool_kv(m->pool), m->table_dev, (int)position, 1, (int)layer, 1,
                          rows, rows + width, 1, 0, status) &&
             pgpu_copy_d2h(s, &st, status, sizeof(int)) && st == 0;
    }
    ph_unlock();
    return ok;
}

int phonon_kv_cache_commit_position(PhononKvCache *cache, size_t position) {
    if (!cache || !cache->keys || position != cache->length || position >= cache->capacity)
        return 0;
    cache->length++;
    return 1;
}

/* ----------------------------------------------------------- primitives -- */

/* Runs one host->device->host primitive on scratch slots 2..4. */
int phonon_rms_norm(const float *input, const float *weight, size_t width, float epsilon,
                    float *output) {
    if (!input || !weight || !output || !width || width > INT_MAX / 4 || !(epsilon > 0.0f) ||
        !isfinite(epsilon) || !ph_all_finite(input, width) || !ph_all_finite(weight, width) ||
        !ph_init())
        return 0;
    ph_lock();
    void *s = ph_stream();
    float *d = ph_scratch(2, 3 * width * sizeof(float));
    int *status = ph_scratch(1, sizeof(int));
    int st = 1;
    int ok = d && status && pgpu_memset(s, status, 0, sizeof(int)) &&
             pgpu_copy_h2d(s, d, input, width * sizeof(float)) &&
             pgpu_copy_h2d(s, d + width, weight, width * sizeof(float)) &&
             pgpu_norm_row(s, d, (int)width, d + width, NULL, epsilon, 1, d + 2 * width, status) &&
             pgpu_copy_d2h(s, &st, status, sizeof(int)) &&
             pgpu_copy_d2h(s, output, d + 2 * width, width * sizeof(float));
    ph_unlock();
    return ok && st == 0;
}

int phonon_layer_norm(const float *input, const float *weight, const float *bias, size_t width,
                      float epsilon, float *output) {
    if (!input || !weight || !bias || !output || !width || width > INT_MAX / 4 ||
        !(epsilon > 0.0f) || !isfinite(epsilon) || !ph_all_finite(input, width) ||
        !ph_all_finite(weight, width) || !ph_all_finite(bias, width) || !ph_init())
        return 0;
    ph_lock();
    void *s = ph_stream();
    float *d = ph_scratch(2, 4 * width * sizeof(float));
    int *status = ph_scratch(1, sizeof(int));
    int st = 1;
    int ok = d && status && pgpu_memset(s, status, 0, sizeof(int)) &&
             pgpu_copy_h2d(s, d, input, width * sizeof(float)) &&
             pgpu_copy_h2d(s, d + width, weight, width * sizeof(float)) &&
             pgpu_copy_h2d(s, d + 2 * width, bias, width * sizeof(float)) &&
             pgpu_norm_row(s, d, (int)width, d + width, d + 2 * width, epsilon, 0, d + 3 * width,
                           status) &&
             pgpu_copy_d2h(s, &st, status, sizeof(int)) &&
             pgpu_copy_d2h(s, output, d + 3 * width, width * sizeof(float));
    ph_unlock();
    return ok && st == 0;
}

int phonon_erf_gelu(float *values, size_t count) {
    if (!values && count)
        return 0;
    if (!count)
        return 1;
    if (!ph_all_finite(values, count) || !ph_init())
        return 0;
    ph_lock();
    void *s = ph_stream();
    float *d = ph_scratch(2, count * sizeof(float));
    int *status = ph_scratch(1, sizeof(int));
    int st = 1;
    int ok = d && status && pgpu_memset(s, status, 0, sizeof(int)) &&
             pgpu_copy_h2d(s, d, values, count * sizeof(float)) &&
             pgpu_gelu(s, d, count, status) && pgpu_copy_d2h(s, &st, status, sizeof(int));
    /* The reference writes values in place up to the first failure; on
     * failure the contents are left as they were. */
    ok = ok && st == 0 && pgpu_copy_d2h(s, values, d, count * sizeof(float));
    ph_unlock();
    return ok;
}

int phonon_rope_interleaved(float *values, size_t width, size_t heads, size_t position,
                            float theta) {
    if (!values || !width || !heads || width % heads || (width / heads) % 2 ||
        !(theta > 0.0f) || !isfinite(theta) || width > INT_MAX / 4)
        return 0;
    const size_t head_width = width / heads;
    float *cos_sin = malloc(head_width * sizeof(float));
    if (!cos_sin)
        return 0;
    ph_rope_row(theta, position, head_width, cos_sin);
    if (!ph_all_finite(cos_sin, head_width) || !ph_all_finite(values, width) || !ph_init()) {
        free(cos_sin);
        return 0;
    }
    ph_lock();
    void *s = ph_stream();
    float *d = ph_scratch(2, (width + head_width) * sizeof(float));
    int *status = ph_scratch(1, sizeof(int));
    int st = 1;
    int ok = d && status && pgpu_memset(s, status, 0, sizeof(int)) &&
             pgpu_copy_h2d(s, d, values, width * sizeof(float)) &&
             pgpu_copy_h2d(s, d + width, cos_sin, head_width * sizeof(float)) &&
             pgpu_rope(s, d, (int)heads, (int)head_width, d + width, status) &&
             pgpu_copy_d2h(s, &st, status, sizeof(int));
    ok = ok && st == 0 && pgpu_copy_d2h(s, values, d, width * sizeof(float));
    ph_unlock();
    free(cos_sin);
    return ok;
}

int phonon_linear_batch(const PhononTensorView *weight, const float *input, size_t rows,
                        size_t columns, const float *bias, float *output, size_t batch) {
    /* Argument contract of src/phonon_transformer.c:253-281. */
    if (!weight || !weight->data || !input || !output || !rows || !columns || !batch ||
        batch > INT_MAX || batch > SIZE_MAX / rows || batch > SIZE_MAX / columns ||
        rows > SIZE_MAX / columns || weight->rank != 2 || weight->shape[0] != rows ||
        weight->shape[1] != columns || weight->byte_count == 0)
        return 0;
    if (batch * rows > SIZE_MAX / sizeof(float) || batch * columns > SIZE_MAX / sizeof(float) ||
        rows > INT_MAX || columns > INT_MAX)
        return 0;
    if (!ph_all_finite(input, batch * columns))
        return 0;
    const size_t elements = rows * columns;
    if (weight->dtype == PHONON_PACK_Q8_0) {
        if (columns % 32 || weight->byte_count != elements / 32 * sizeof(PhononQ8Block))
            return 0;
        const size_t in_bytes = batch * columns * sizeof(float);
        const size_t out_bytes = batch * rows * sizeof(float);
        if (ph_overlap(input, in_bytes, output, out_bytes) ||
            ph_overlap(weight->data, weight->byte_count, output, out_bytes))
            return 0;
    } else if (weight->dtype != PHONON_PACK_BF16 ||
               weight->byte_count != elements * sizeof(uint16_t)) {
        return 0;
    }
    if (bias && !ph_all_finite(bias, rows))
        return 0;
    if (!ph_init())
        return 0;
    ph_lock();
    void *s = ph_stream();
    pgpu_matrix w;
    void *wdev = NULL;
    int ok = ph_matrix_upload(weight, rows, columns, &w, &wdev);
    const size_t prow = w.rows, pcol = w.columns, pbatch = (batch + 15) / 16 * 16;
    float *x = NULL, *y = NULL, *b = NULL, *host = NULL;
    uint16_t *xs = NULL;
    int *status = ph_scratch(1, sizeof(int));
    if (ok) {
        x = ph_scratch(2, batch * pcol * sizeof(float));
        y = ph_scratch(3, batch * prow * sizeof(float));
        b = bias ? ph_scratch(4, prow * sizeof(float)) : NULL;
        xs = ph_scratch(5, pbatch * pcol * 3 * sizeof(uint16_t));
        host = calloc(batch * (pcol > prow ? pcol : prow), sizeof(float));
        ok = x && y && xs && status && host && (!bias || b);
    }
    if (ok) {
        for (size_t i = 0; i < batch; i++)
            memcpy(host + i * pcol, input + i * columns, columns * sizeof(float));
        ok = pgpu_memset(s, status, 0, sizeof(int)) &&
             pgpu_memset(s, xs, 0, pbatch * pcol * 3 * sizeof(uint16_t)) &&
             pgpu_copy_h2d(s, x, host, batch * pcol * sizeof(float));
        if (ok && bias) {
            memset(host, 0, prow * sizeof(float));
            memcpy(host, bias, rows * sizeof(float));
            ok = pgpu_copy_h2d(s, b, host, prow * sizeof(float));
        }
    }
    int st = 1;
    const pgpu_gemm_input in = {.split = xs};
    ok = ok && pgpu_split_rows(s, x, (int)batch, (int)pcol, xs, status) &&
         pgpu_gemm_store(s, &w, &in, (int)batch, b, y, (int)prow, status) &&
         pgpu_copy_d2h(s, &st, status, sizeof(int)) &&
         pgpu_copy_d2h(s, host, y, batch * prow * sizeof(float));
    if (ok && st == 0)
        for (size_t i = 0; i < batch; i++)
            memcpy(output + i * rows, host + i * prow, rows * sizeof(float));
    (void)pgpu_stream_sync(s);
    pgpu_free(wdev);
    ph_unlock();
    free(host);
    return ok && st == 0 && ph_all_finite(output, batch * rows);
}

int phonon_linear(const PhononTensorView *weight, const float *input, size_t rows, size_t columns,
                  const float *bias, float *output) {
    return phonon_linear_batch(weight, input, rows, columns, bias, output, 1);
}

/* --------------------------------------------------------- decode steps -- */

/* Runs model layers [0, model_layers) as pool layers [pool_first, ...) for
 * one stream at `position`, reading `input` (host [512]) and writing
 * `output` (host [512]); polls `cancel` before every layer and after the
 * last. Copies the appended K/V rows back into the cache's host arrays. */
static int run_position(const PhononFlowModel *model, Mirror *m, PhononKvCache *cache,
                        size_t pool_first, size_t position, const float *input, float theta,
                        float *output, PhononCancelPoll cancel, void *context, int *cancelled) {
    *cancelled = 0;
    const size_t layers = phonon_flow_model_layers(model);
    if (!m->batch && !phonon_flow_batch_create(model, m->pool, 1, m->positions, &m->batch))
        return ph_fail("decode step: batch creation failed");
    PhononFlowBatch *b = m->batch;
    void *s = ph_batch_stream(b);
    float *in = ph_batch_in(b), *out = ph_batch_out(b);
    if (!ph_batch_bind_model(b, model) || !ph_batch_set_single(b, position, m->table_dev) ||
        !pgpu_copy_h2d(s, in, input, PHONON_FLOW_WIDTH * sizeof(float)))
        return ph_fail("decode step: setting up the stream failed");
    for (size_t l = 0; l < layers; l++) {
        if (cancel && cancel(context)) {
            *cancelled = 1;
            (void)ph_batch_status(b);
            return 0;
        }
        if (!ph_batch_enqueue_layers(b, l, 1, pool_first, l ? out : in, out, theta))
            return ph_fail("decode step: enqueueing a layer failed");
    }
    if (cancel && cancel(context)) {
        *cancelled = 1;
        (void)ph_batch_status(b);
        return 0;
    }
    float *rows = ph_batch_scratch_rows(b);
    if (!pgpu_kv_copy(s, ph_pool_kv(m->pool), m->table_dev, (int)position, 1, (int)pool_first,
                      (int)layers, rows, rows + layers * PH_WIDTH, 1, 1,
                      ph_batch_status_word(b))) {
        (void)ph_batch_status(b);
        return ph_fail("decode step: copying appended rows failed");
    }
    const int clean = ph_batch_status(b);
    float *host_rows = malloc(2 * layers * PH_WIDTH * sizeof(float));
    int ok = host_rows &&
             pgpu_copy_d2h(s, host_rows, rows, 2 * layers * PH_WIDTH * sizeof(float)) &&
             pgpu_copy_d2h(s, output, out, PHONON_FLOW_WIDTH * sizeof(float));
    if (ok)
        for (size_t l = 0; l < layers; l++) {
            const size_t offset = ((pool_first + l) * cache->capacity + position) * PH_WIDTH;
            memcpy(cache->keys + offset, host_rows + l * PH_WIDTH, PH_WIDTH * sizeof(float));
            memcpy(cache->values + offset, host_rows + (layers + l) * PH_WIDTH,
                   PH_WIDTH * sizeof(float));
        }
    free(host_rows);
    if (!ok)
        return ph_fail("decode step: reading results failed");
    if (!clean)
        return ph_fail("decode step: non-finite value or uncovered position on the device");
    return ph_all_finite(output, PHONON_FLOW_WIDTH) ||
           ph_fail("decode step: non-finite output");
}

/* Prefill of positions [0, length) for the stream of `m`: chunks of up to
 * PH_PREFILL_CHUNK positions, each run through all layers in one batched
 * pass (phonon_flow_batch_prefill_device semantics), polling `cancel` before
 * every layer and after the last; then the appended K/V rows are copied back
 * into the cache's host arrays and `output` receives the last position's
 * output (src/phonon_transformer.c:692). */
static int run_prefill(const PhononFlowModel *model, Mirror *m, PhononKvCache *cache,
                       const float *input, size_t length, float theta, float *output,
                       PhononCancelPoll cancel, void *context, int *cancelled) {
    *cancelled = 0;
    const size_t layers = phonon_flow_model_layers(model);
    const size_t chunk = m->positions < PH_PREFILL_CHUNK ? m->positions : PH_PREFILL_CHUNK;
    if (!m->prefill && !phonon_flow_batch_create(model, m->pool, chunk, m->positions, &m->prefill))
        return ph_fail("prefill: batch creation failed");
    PhononFlowBatch *b = m->prefill;
    void *s = ph_batch_stream(b);
    float *in = ph_batch_in(b), *out = ph_batch_out(b);
    if (!ph_batch_bind_model(b, model))
        return ph_fail("prefill: binding the model failed");
    size_t last = 0;
    for (size_t start = 0; start < length; start += chunk) {
        const size_t n = length - start < chunk ? length - start : chunk;
        if (!ph_batch_set_prefill(b, 1, &start, &n, m->table_dev) ||
            !pgpu_copy_h2d(s, in, input + start * PH_WIDTH, n * PH_WIDTH * sizeof(float)))
            return ph_fail("prefill: setting up the positions failed");
        for (size_t l = 0; l < layers; l++) {
            if (cancel && cancel(context)) {
                *cancelled = 1;
                (void)ph_batch_status(b);
                return 0;
            }
            if (!ph_batch_enqueue_layers(b, l, 1, 0, l ? out : in, out, theta))
                return ph_fail("prefill: enqueueing a layer failed");
        }
        if (!ph_batch_status(b))
            return ph_fail("prefill: non-finite value or uncovered position on the device");
        last = n - 1;
    }
    if (cancel && cancel(context)) {
        *cancelled = 1;
        return 0;
    }
    if (!pgpu_copy_d2h(s, output, out + last * PH_WIDTH, PH_WIDTH * sizeof(float)) ||
        !phonon_kv_pool_read(m->pool, m->table_host, m->table_len, 0, length, cache->keys,
                             cache->values, cache->capacity))
        return ph_fail("prefill: reading results failed");
    return ph_all_finite(output, PHONON_FLOW_WIDTH) || ph_fail("prefill: non-finite output");
}

/* Model for `layers` layers of `weights`: the registered device copy, or a
 * fresh upload owned by the caller (*owned). */
static const PhononFlowModel *model_for(const PhononFlowLayerWeights *weights, size_t layers,
                                        PhononFlowModel **owned) {
    *owned = NULL;
    const PhononFlowModel *m = ph_registered_model(weights, layers);
    if (m)
        return m;
    if (!phonon_flow_model_create(weights, layers, owned)) {
        ph_fail("decode step: weights rejected (shape, dtype, size or non-finite value) or "
                "upload failed");
        return NULL;
    }
    return *owned;
}

/* The device weights and the cache's device copy, found under the library
 * lock; the copy is returned locked (its own lock), so steps of different
 * caches run concurrently. NULL if either is missing. */
static Mirror *acquire(const PhononFlowLayerWeights *weights, size_t layers,
                       const PhononKvCache *cache, PhononFlowModel **owned,
                       const PhononFlowModel **model) {
    ph_lock();
    *model = model_for(weights, layers, owned);
    Mirror *m = *model ? mirror_get(cache) : NULL;
    ph_unlock();
    if (m)
        pthread_mutex_lock(&m->lock);
    else if (*owned) {
        ph_lock();
        phonon_flow_model_destroy(*owned);
        *owned = NULL;
        ph_unlock();
    }
    return m;
}

/* Ends a step: a weight upload of this call is freed once the batch that
 * used it has finished. */
static void release(Mirror *m, PhononFlowBatch *used, PhononFlowModel *owned) {
    if (!m)
        return;
    if (used && owned)
        (void)ph_batch_status(used);
    pthread_mutex_unlock(&m->lock);
    if (owned) {
        ph_lock();
        phonon_flow_model_destroy(owned);
        ph_unlock();
    }
}

int phonon_flow_layer_step(const PhononFlowLayerWeights *weights, PhononKvCache *cache,
                           size_t layer, size_t position, const float input[PHONON_FLOW_WIDTH],
                           float theta, float output[PHONON_FLOW_WIDTH]) {
    if (!weights || !cache || !input || !output || layer >= PHONON_FLOW_LAYERS ||
        position >= cache->capacity || position >= PHONON_FLOW_MAX_POSITIONS ||
        cache->length != position || !cache->keys || !cache->values ||
        !ph_all_finite(input, PHONON_FLOW_WIDTH) || !ph_init())
        return 0;
    PhononFlowModel *owned = NULL;
    const PhononFlowModel *model;
    Mirror *m = acquire(weights, 1, cache, &owned, &model);
    int cancelled = 0;
    float result[PHONON_FLOW_WIDTH];
    const int ok = m && run_position(model, m, cache, layer, position, input, theta, result, NULL,
                                     NULL, &cancelled);
    release(m, m ? m->batch : NULL, owned);
    if (ok)
        memcpy(output, result, sizeof(result));
    return ok;
}

int phonon_flow_stack_step_cancel(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                                  PhononKvCache *cache, size_t position, const float input[512],
                                  float theta, float output[512], PhononCancelPoll cancel,
                                  void *context) {
    if (!weights || !cache || !input || !output || position != cache->length ||
        position >= cache->capacity)
        return 0;
    if (position >= PHONON_FLOW_MAX_POSITIONS || !cache->keys || !cache->values ||
        !ph_all_finite(input, PHONON_FLOW_WIDTH) || !ph_init())
        return 0;
    PhononFlowModel *owned = NULL;
    const PhononFlowModel *model;
    Mirror *m = acquire(weights, PHONON_FLOW_LAYERS, cache, &owned, &model);
    int cancelled = 0;
    float result[PHONON_FLOW_WIDTH];
    int ok = m && run_position(model, m, cache, 0, position, input, theta, result, cancel,
                               context, &cancelled);
    release(m, m ? m->batch : NULL, owned);
    if (cancelled) {
        phonon_kv_cache_reset(cache);
        return 0;
    }
    if (!ok || !phonon_kv_cache_commit_position(cache, position))
        return 0;
    memcpy(output, result, sizeof(result));
    return 1;
}

int phonon_flow_stack_step(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                           PhononKvCache *cache, size_t position, const float input[512],
                           float theta, float output[512]) {
    return phonon_flow_stack_step_cancel(weights, cache, position, input, theta, output, NULL,
                                         NULL);
}

int phonon_flow_stack_prefill_cancel(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                                     PhononKvCache *cache, const float *input, size_t length,
                                     float theta, float output[512], PhononCancelPoll cancel,
                                     void *context) {
    /* Argument contract of src/phonon_transformer.c:622-626. */
    if (!weights || !cache || !cache->keys || !cache->values || !input || !output || !length ||
        length > PHONON_FLOW_MAX_POSITIONS || length > cache->capacity || cache->length ||
        !isfinite(theta) || theta <= 0.0f || length > SIZE_MAX / (6144 * sizeof(float)))
        return 0;
    if (!ph_all_finite(input, length * PHONON_FLOW_WIDTH) || !ph_init()) {
        phonon_kv_cache_reset(cache);
        return 0;
    }
    PhononFlowModel *owned = NULL;
    const PhononFlowModel *model;
    Mirror *m = acquire(weights, PHONON_FLOW_LAYERS, cache, &owned, &model);
    int cancelled = 0;
    float result[PHONON_FLOW_WIDTH];
    const int ok = m && run_prefill(model, m, cache, input, length, theta, result, cancel,
                                    context, &cancelled);
    release(m, m ? m->prefill : NULL, owned);
    if (!ok || cancelled) {
        phonon_kv_cache_reset(cache);
        return 0;
    }
    memcpy(output, result, sizeof(result));
    cache->length = length;
    return 1;
}

int phonon_flow_stack_prefill(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                              PhononKvCache *cache, const float *input, size_t length, float theta,
                              float output[512]) {
    return phonon_flow_stack_prefill_cancel(weights, cache, input, length, theta, output, NULL,
                                            NULL);
}

/* ------------------------------------------------------------ test seam -- */

int phonon_attention_test(const float query[64], const float *keys, const float *values,
                          size_t count, size_t stride, float output[64]) {
    if (!query || !keys || !values || !output || !count || count > PHONON_FLOW_MAX_POSITIONS ||
        stride < 64 || stride > INT_MAX || !ph_init())
        return 0;
    for (size_t i = 0; i < count; i++)
        if (!ph_all_finite(keys + i * stride, 64) || !ph_all_finite(values + i * stride, 64))
            return 0;
    if (!ph_all_finite(query, 64))
        return 0;
    const size_t table_len = (count + 15) / 16;
    PhononKvPool *pool = NULL;
    int32_t *table = malloc(table_len * sizeof(int32_t));
    float *k = calloc(count * PH_WIDTH, sizeof(float)), *v = calloc(count * PH_WIDTH, sizeof(float));
    float q[PH_WIDTH] = {0};
    int ok = table && k && v && phonon_kv_pool_create(1, table_len, &pool) &&
             phonon_kv_pool_alloc(pool, table_len, table);
    if (ok) {
        for (size_t i = 0; i < count; i++) {
            memcpy(k + i * PH_WIDTH, keys + i * stride, 64 * sizeof(float));
            memcpy(v + i * PH_WIDTH, values + i * stride, 64 * sizeof(float));
        }
        /* Scores are (q.k)/8: the power-of-two scale folds into q exactly. */
        for (size_t d = 0; d < 64; d++)
            q[d] = query[d] * 0.125f;
        ok = phonon_kv_pool_write(pool, table, table_len, 0, count, k, v, count);
    }
    ph_lock();
    void *s = ph_stream();
    const int splits = (int)((count + PH_SPLIT_KEYS - 1) / PH_SPLIT_KEYS);
    float *dq = ok ? ph_scratch(2, 2 * PH_WIDTH * sizeof(float)) : NULL;
    int32_t *dt = ok ? ph_scratch(3, (table_len + 1) * sizeof(int32_t)) : NULL;
    /* Partials of one stream, head 0: slots j = 0 .. splits-1. */
    float *part = ok ? ph_scratch(4, (size_t)splits * PH_HEADS * 66 * sizeof(float)) : NULL;
    int *words = ok ? ph_scratch(5, sizeof(int)) : NULL;
    int st = 1;
    if (ok && dq && dt && part && words) {
        const int32_t position = (int32_t)(count - 1);
        pgpu_attention_scratch scratch = {part, part + (size_t)splits * PH_HEADS * 64, 1,
                                          splits};
        ok = pgpu_memset(s, words, 0, sizeof(int)) &&
             pgpu_copy_h2d(s, dq, q, PH_WIDTH * sizeof(float)) &&
             pgpu_copy_h2d(s, dt, table, table_len * sizeof(int32_t)) &&
             pgpu_copy_h2d(s, dt + table_len, &position, sizeof(int32_t)) &&
             pgpu_attention(s, dq, ph_pool_kv(pool), 0, dt, (int)table_len, dt + table_len, 1, 1,
                            splits, &scratch, words) &&
             pgpu_attention_merge(s, &scratch, dt + table_len, 1, 1, splits, dq + PH_WIDTH, NULL,
                                  words) &&
             pgpu_copy_d2h(s, &st, words, sizeof(int)) &&
             pgpu_copy_d2h(s, output, dq + PH_WIDTH, 64 * sizeof(float));
    } else {
        ok = 0;
    }
    ph_unlock();
    phonon_kv_pool_destroy(pool);
    free(table);
    free(k);
    free(v);
    return ok && st == 0 && ph_all_finite(output, 64);
}
