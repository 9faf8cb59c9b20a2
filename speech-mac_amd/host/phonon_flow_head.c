/* Flow head on the GPU (phonon_sampler.h): src/phonon_sampler.c:280-401 as
 * a chain of 15 launches over B streams (pgpu_head.hip):
 *   front   s_y = SiLU(cond_embed(condition) + tsum)    split fragments
 *           eos = out_eos . condition + bias            (optional)
 *           noise = raw * sqrt(T)                        [B][32] + fragments
 *   mod     mod = [adaLN_0 .. adaLN_5 | final adaLN](s_y) [B][6*1536 + 1024]
 *           x   = input_proj(noise)                      [B][512]
 *   6 x     u = SiLU(mlp_b0(LN(x)*(1 + scale_b) + shift_b))
 *           x += gate_b * mlp_b1(u)
 *   final   latent = noise + final(LN(x)*(1 + scale_f) + shift_f)
 * SiLU(y) is the same for all seven adaLN projections (they read only the
 * condition and the time embeddings), so they run as one 10240-row
 * projection. The time embeddings of the LSD step (s = 0, t = 1) do not
 * depend on the stream: tsum = 0.5 (time_0(0) + time_1(1)) is computed once
 * on the device when the head is created. */
#include "phonon_sampler.h"
#include "ph_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum {
    HB = PHONON_FLOW_HEAD_BLOCKS,
    /* The fused chain reads its 8 partials of every live stream of a tile
     * in each of the tile's 8 work-groups (16 KB per stream): it is faster
     * than two launches per block only for the smallest steps (B = 1, 2:
     * 1-4 us of 72; B = 4: 3 us slower, B = 64: 18 us slower). */
    FUSED_AUTO_STREAMS = 2,
    /* The tagged one-launch step: each consumer polls its operand words
     * itself, so the poll traffic grows with the live streams of a tile; it
     * is the fastest form at B = 1 and 2 (63 / 68 us against 72 / 73 for
     * the chain, graph replay) and slower from 4 streams on (B = 16: 117 vs
     * 74 us). */
    TAGGED_AUTO_STREAMS = 2,
    ADA = 3 * PH_WIDTH,              /* rows of one block's adaLN */
    FINAL_ADA = 2 * PH_WIDTH,
    MOD = HB * ADA + FINAL_ADA,      /* 10240 modulation columns */
    LAT = PHONON_LATENT_WIDTH,
    EOS_ROWS = 16,                   /* the EOS row padded to one row tile */
};

struct PhononFlowHeadDevice {
    pgpu_matrix input, cond, ada, mlp[HB][2], final, eos, time_w[2][2];
    void *mats[7 + 2 * HB + 4];
    size_t nmats;
    float *vec; /* every bias / norm / frequency / alpha vector, and tsum */
    float *b_input, *b_cond, *b_ada, *b_mlp[HB][2], *b_final, *b_eos, *b_time[2][2];
    float *norm_w[HB], *norm_b[HB], *freqs[2], *alpha[2];
    float *tsum_lsd, *tsum, *time_out; /* time_out: [2][512] */
    float *ones;                       /* [32] of 1.0f: the Euler update's gate */
    float *out_norm;                   /* (frame) [2][512] LayerNorm weight, bias */
    pgpu_matrix input_linear;          /* (frame) [512][32] latent embedding */
    void *input_linear_dev;
    int has_frame;
    size_t cap;                        /* streams, a multiple of 16 */
    void *buffers;
    float *noise, *x, *mod, *velocity, *eos_rows, *stage;
    /* The fused chain (pgpu_head_block): the second x buffer and two sets
     * of a block's 8 partials [8][cap][512], used alternately. fused: 1
     * always, 0 never, -1 (the default) for steps of at most
     * FUSED_AUTO_STREAMS streams. */
    int fused;
    float *x2, *parts[2];
    uint16_t *noise_split, *silu_split, *first_split, *time_split, *time_hidden;
    int has_eos;
    int *status;
    void *stream, *own_stream; /* the stream in use; the one the head created */
    struct {
        void *exec;
        size_t streams;
        const float *conditions, *raw_noise, *embed;
        float temperature;
        float *latents, *eos_logits, *next;
    } graphs[2];
    size_t graph_victim;
    int use_graph; /* 1: replay a captured graph; 0: launch each kernel directly;
                      -1 (the default): a graph for the chain of launches, the
                      one-launch forms launched directly */
    /* One-launch step (pgpu_head_flow): x of every block, u of every block,
     * counters, and the task lists built so far. */
    int one_launch; /* 0: the chain, 1: one launch, 2: one launch with tagged hand-offs,
                       -1 (the default): 2 for steps of at most TAGGED_AUTO_STREAMS
                       streams, else 0 */
    unsigned wait_us;
    /* Tagged one-launch step: x and u rows as tagged words ([7 + 6][cap][512],
     * allocated on first use), the device tag word, and the tag the next
     * launch uses (tracked here so that the words are cleared before the
     * 32-bit tag would wrap). */
    uint64_t *tagged_rows;
    unsigned *tag_word;
    uint64_t tag_next;
    void *flow_buffers;
    float *fx;
    uint16_t *fu, *latent_split;
    unsigned *counters;
    size_t counter_count;
    struct {
        int tiles, eos, embed, tasks;
        uint32_t *dev;
    } lists[8];
    size_t nlists;
};

static size_t split_elems(size_t streams, size_t k_cols) {
    return (streams + 15) / 16 * (k_cols / 32) * 1536;
}

/* A BF16 [count] vector view into `dst` (fp32). */
static int vec_view(const PhononTensorView *view, size_t count, float *dst) {
    return ph_vector_decode(view, count, dst);
}

static int upload(PhononFlowHeadDevice *h, const PhononTensorView *view, size_t rows,
                  size_t columns, pgpu_matrix *dst) {
    void *dev = NULL;
    if (!ph_matrix_upload(view, rows, columns, dst, &dev))
        return 0;
    h->mats[h->nmats++] = dev;
    return 1;
}

/* The seven adaLN matrices as one BF16 [10240][512] matrix. */
static int upload_ada(PhononFlowHeadDevice *h, const PhononFlowHead *head) {
    uint16_t *all = malloc((size_t)MOD * PH_WIDTH * sizeof(uint16_t));
    if (!all)
        return 0;
    int ok = 1;
    for (size_t b = 0; ok && b <= HB; b++) {
        const PhononTensorView *v = b < HB ? &head->block_ada_weight[b] : &head->final_ada_weight;
        const size_t rows = b < HB ? ADA : FINAL_ADA;
        ok = v->data && v->dtype == PHONON_PACK_BF16 && v->rank == 2 && v->shape[0] == rows &&
             v->shape[1] == PH_WIDTH && v->byte_count == rows * PH_WIDTH * sizeof(uint16_t);
        if (ok)
            memcpy(all + b * ADA * PH_WIDTH, v->data, rows * PH_WIDTH * sizeof(uint16_t));
    }
    PhononTensorView view = {.dtype = PHONON_PACK_BF16,
                             .rank = 2,
                             .shape = {MOD, PH_WIDTH},
                             .data = all,
                             .byte_count = (size_t)MOD * PH_WIDTH * sizeof(uint16_t)};
    ok = ok && upload(h, &view, MOD, PH_WIDTH, &h->ada);
    free(all);
    return ok;
}

/* Device float vectors, laid out in one allocation. */
static int upload_vectors(PhononFlowHeadDevice *h, const PhononFlowHead *head,
                          const PhononTensorView *eos_bias) {
    const size_t total = 2 * PH_WIDTH + MOD + HB * 2 * PH_WIDTH + LAT + EOS_ROWS +
                         2 * 2 * PH_WIDTH + HB * 2 * PH_WIDTH + 2 * 128 + 2 * PH_WIDTH +
                         2 * PH_WIDTH + 2 * PH_WIDTH + LAT;
    float *host = calloc(total, sizeof(float));
    float *dev = host ? pgpu_malloc(total * sizeof(float)) : NULL;
    if (!dev) {
        free(host);
        return 0;
    }
    h->vec = dev;
    size_t at = 0;
    int ok = 1;
#define SLOT(ptr, count) ((ptr) = dev + at, at += (count), host + at - (count))
#define TAKE(ptr, count, view) (ok = ok && vec_view((view), (count), SLOT(ptr, count)))
    TAKE(h->b_input, PH_WIDTH, &head->input_bias);
    TAKE(h->b_cond, PH_WIDTH, &head->cond_bias);
    float *ada = SLOT(h->b_ada, MOD);
    for (size_t b = 0; ok && b < HB; b++)
        ok = vec_view(&head->block_ada_bias[b], ADA, ada + b * ADA);
    ok = ok && vec_view(&head->final_ada_bias, FINAL_ADA, ada + HB * ADA);
    for (size_t b = 0; b < HB; b++)
        for (size_t j = 0; j < 2; j++)
            TAKE(h->b_mlp[b][j], PH_WIDTH, &head->block_mlp_bias[b][j]);
    TAKE(h->b_final, LAT, &head->final_bias);
    float *eos = SLOT(h->b_eos, EOS_ROWS);
    if (eos_bias)
        ok = ok && vec_view(eos_bias, 1, eos);
    for (size_t i = 0; i < 2; i++)
        for (size_t j = 0; j < 2; j++)
            TAKE(h->b_time[i][j], PH_WIDTH, &head->time_bias[i][j]);
    for (size_t b = 0; b < HB; b++) {
        TAKE(h->norm_w[b], PH_WIDTH, &head->block_norm_weight[b]);
        TAKE(h->norm_b[b], PH_WIDTH, &head->block_norm_bias[b]);
    }
    for (size_t i = 0; i < 2; i++) {
        TAKE(h->freqs[i], 128, &head->time_freqs[i]);
        TAKE(h->alpha[i], PH_WIDTH, &head->time_alpha[i]);
    }
    (void)SLOT(h->tsum_lsd, PH_WIDTH);
    (void)SLOT(h->tsum, PH_WIDTH);
    (void)SLOT(h->time_out, 2 * PH_WIDTH);
    float *ones = SLOT(h->ones, LAT);
    for (size_t i = 0; i < LAT; i++)
        ones[i] = 1.0f;
#undef TAKE
#undef SLOT
    ok = ok && at == total && pgpu_copy_h2d(h->stream, dev, host, total * sizeof(float)) &&
         pgpu_stream_sync(h->stream);
    free(host);
    return ok;
}

/* The buffers of the one-launch step for up to h->cap streams. */
static int alloc_flow_buffers(PhononFlowHeadDevice *h) {
    const size_t cap = h->cap, tiles = cap / 16;
    const size_t floats = (HB + 1) * cap * PH_WIDTH;
    const size_t halves = HB * split_elems(cap, PH_WIDTH) + split_elems(cap, LAT);
    const size_t counters = tiles * PGPU_HEADC_KINDS * PGPU_HEAD_COUNTER_STRIDE;
    const size_t bytes = floats * sizeof(float) + halves * sizeof(uint16_t) +
                         counters * sizeof(unsigned);
    char *p = pgpu_malloc(bytes);
    if (!p || !pgpu_memset(h->stream, p, 0, bytes)) {
        pgpu_free(p);
        return 0;
    }
    h->flow_buffers = p;
    h->fx = (float *)p;
    h->fu = (uint16_t *)(h->fx + floats);
    h->latent_split = h->fu + HB * split_elems(cap, PH_WIDTH);
    h->counters = (unsigned *)(h->latent_split + split_elems(cap, LAT));
    h->counter_count = counters;
    return 1;
}

/* The one-launch task list (pgpu_head_flow): every task after the tasks it
 * waits for. The modulation rows of block b + 1 are listed between block
 * b's MLP_IN and MLP_OUT tasks, so that they are computed while the chain
 * works on block b. Returns the number of tasks (with out == NULL: only
 * counts them; 0 if `capacity` is too small). */
int pgpu_head_flow_schedule(uint32_t *out, int capacity, int tiles, int with_eos,
                            int with_embed) {
    if (tiles <= 0 || tiles > 255 || capacity < 0)
        return 0;
    int n = 0;
#define PUT(kind, block, tile, index)                                                      \
    do {                                                                                   \
        if (out && n < capacity)                                                           \
            out[n] = PGPU_HEAD_TASK(kind, block, tile, index);                             \
        n++;                                                                               \
    } while (0)
    const int groups512 = (PH_WIDTH / 16 + 3) / 4, rows512 = PH_WIDTH / 16;
    const int ada_block = ADA / 64, ada_final = FINAL_ADA / 64;
    for (int t = 0; t < tiles; t++) {
        for (int i = 0; i < groups512; i++)
            PUT(PGPU_HEAD_COND, 0, t, i);
        if (with_eos)
            PUT(PGPU_HEAD_EOS, 0, t, 0);
        PUT(PGPU_HEAD_NOISE, 0, t, 0);
    }
    for (int t = 0; t < tiles; t++)
        for (int i = 0; i < rows512; i++)
            PUT(PGPU_HEAD_INPUT, 0, t, i);
    for (int t = 0; t < tiles; t++)
        for (int i = 0; i < ada_block; i++)
            PUT(PGPU_HEAD_ADA, 0, t, i);
    for (int t = 0; t < tiles; t++)
        for (int i = 0; i < groups512; i++)
            PUT(PGPU_HEAD_MLP_IN, 0, t, i);
    for (int b = 0; b < HB; b++) {
        const int nb = b + 1, groups = nb < HB ? ada_block : ada_final;
        for (int t = 0; t < tiles; t++)
            for (int i = 0; i < groups; i++)
                PUT(PGPU_HEAD_ADA, 0, t, nb * ada_block + i);
        for (int t = 0; t < tiles; t++)
            for (int i = 0; i < rows512; i++)
                PUT(PGPU_HEAD_MLP_OUT, b, t, i);
        if (nb < HB)
            for (int t = 0; t < tiles; t++)
                for (int i = 0; i < groups512; i++)
                    PUT(PGPU_HEAD_MLP_IN, nb, t, i);
    }
    for (int t = 0; t < tiles; t++)
        PUT(PGPU_HEAD_FINAL, 0, t, 0);
    if (with_embed)
        for (int t = 0; t < tiles; t++)
            for (int i = 0; i < rows512; i++)
                PUT(PGPU_HEAD_EMBED, 0, t, i);
#undef PUT
    return !out || n <= capacity ? n : 0;
}

/* The device copy of the task list for (tiles, eos, embed), built once. */
static const uint32_t *flow_list(PhononFlowHeadDevice *h, int tiles, int eos, int embed,
                                 int *tasks) {
    for (size_t i = 0; i < h->nlists; i++)
        if (h->lists[i].tiles == tiles && h->lists[i].eos == eos && h->lists[i].embed == embed) {
            *tasks = h->lists[i].tasks;
            return h->lists[i].dev;
        }
    if (h->nlists == sizeof(h->lists) / sizeof(h->lists[0]))
        return NULL;
    const int n = pgpu_head_flow_schedule(NULL, 0, tiles, eos, embed);
    uint32_t *host = n > 0 ? malloc((size_t)n * sizeof(uint32_t)) : NULL;
    uint32_t *dev = host ? pgpu_malloc((size_t)n * sizeof(uint32_t)) : NULL;
    const int ok = dev && pgpu_head_flow_schedule(host, n, tiles, eos, embed) == n &&
                   pgpu_copy_h2d(h->stream, dev, host, (size_t)n * sizeof(uint32_t)) &&
                   pgpu_stream_sync(h->stream);
    free(host);
    if (!ok) {
        pgpu_free(dev);
        return NULL;
    }
    h->lists[h->nlists].tiles = tiles;
    h->lists[h->nlists].eos = eos;
    h->lists[h->nlists].embed = embed;
    h->lists[h->nlists].tasks = n;
    h->lists[h->nlists].dev = dev;
    h->nlists++;
    *tasks = n;
    return dev;
}

static int alloc_buffers(PhononFlowHeadDevice *h, size_t streams) {
    const size_t cap = (streams + 15) / 16 * 16;
    const size_t floats =
        cap * (LAT + PH_WIDTH + MOD + LAT + EOS_ROWS + PH_WIDTH + 2 * 8 * PH_WIDTH) + PH_WIDTH +
        LAT;
    const size_t halves = split_elems(cap, LAT) + 2 * split_elems(cap, PH_WIDTH) +
                          split_elems(16, 256) + split_elems(16, PH_WIDTH);
    const size_t bytes = floats * sizeof(float) + halves * sizeof(uint16_t);
    char *p = pgpu_malloc(bytes);
    if (!p || !pgpu_memset(h->stream, p, 0, bytes))
        return 0;
    h->buffers = p;
    h->cap = cap;
    float *f = (float *)p;
    h->noise = f, f += cap * LAT;
    h->x = f, f += cap * PH_WIDTH;
    h->x2 = f, f += cap * PH_WIDTH;
    h->parts[0] = f, f += 8 * cap * PH_WIDTH;
    h->parts[1] = f, f += 8 * cap * PH_WIDTH;
    h->mod = f, f += cap * MOD;
    h->velocity = f, f += cap * LAT;
    h->eos_rows = f, f += cap * EOS_ROWS;
    h->stage = f, f += PH_WIDTH + LAT;
    uint16_t *u = (uint16_t *)f;
    h->noise_split = u, u += split_elems(cap, LAT);
    h->silu_split = u, u += split_elems(cap, PH_WIDTH);
    h->first_split = u, u += split_elems(cap, PH_WIDTH);
    h->time_split = u, u += split_elems(16, 256);
    h->time_hidden = u;
    return 1;
}

/* tsum = 0.5 (time_0(s) + time_1(t)) (src/phonon_sampler.c:280-305, 318-319). */
static int enqueue_tsum(PhononFlowHeadDevice *h, float s, float t, float *tsum) {
    for (int which = 0; which < 2; which++) {
        const pgpu_gemm_input phase = {.split = h->time_split};
        const pgpu_gemm_input hidden = {.split = h->time_hidden};
        if (!pgpu_head_time_phase(h->stream, h->freqs[which], which ? t : s, h->time_split,
                                  h->status) ||
            !pgpu_gemm_silu_split(h->stream, &h->time_w[which][0], &phase, 1, h->b_time[which][0],
                                  NULL, h->time_hidden, h->status) ||
            !pgpu_gemm_store(h->stream, &h->time_w[which][1], &hidden, 1, h->b_time[which][1],
                             h->time_out + which * PH_WIDTH, PH_WIDTH, h->status))
            return 0;
    }
    return pgpu_head_time_sum(h->stream, h->time_out, h->time_out + PH_WIDTH, h->alpha[0],
                              h->alpha[1], tsum, h->status);
}

/* The head for n streams: conditions [n][512], raw [n][32] scaled by `scale`
 * (out_split: the latent's split fragments too, lsd only)
 * into the state (the noise of an LSD step, or the normalized state itself
 * with scale 1). Writes the latent noise + velocity (lsd) or the velocity to
 * out [n][32] and, if eos, the EOS logits. The cancel poll runs before each
 * block and before the final layer. */
static int enqueue_head(PhononFlowHeadDevice *h, size_t n, const float *conditions,
                        const float *norm, const float *raw, float scale, const float *tsum,
                        int lsd, float *out, uint16_t *out_split, float *eos,
                        PhononCancelPoll cancel, void *context) {
    void *st = h->stream;
    const int B = (int)n;
    const pgpu_gemm_input first = {.split = h->first_split};
    if (!pgpu_head_front(st, &h->cond, conditions, B, norm, norm ? norm + PH_WIDTH : NULL,
                         h->b_cond, tsum, h->silu_split,
                         eos ? &h->eos : NULL, h->b_eos, h->eos_rows, EOS_ROWS, raw, scale,
                         h->noise, h->noise_split, h->status) ||
        !pgpu_head_mod(st, &h->ada, h->silu_split, B, h->b_ada, h->mod, MOD, &h->input,
                       h->noise_split, h->b_input, h->x, h->status))
        return 0;
    if (h->fused > 0 || (h->fused < 0 && n <= FUSED_AUTO_STREAMS)) {
        /* x_0 (the input projection) is in xs[0]; block b >= 1 reads
         * x_(b-1) from xs[(b-1) % 2] and block b-1's partials from
         * parts[(b-1) % 2], and writes x_b to xs[b % 2] and its partials to
         * parts[b % 2]; the final layer reads x_5 and block 5's partials. */
        float *xs[2] = {h->x, h->x2};
        pgpu_head_parts prev = {.ld_parts = (int)h->cap, .ld_gate = MOD};
        for (size_t b = 0; b < HB; b++) {
            if (cancel && cancel(context))
                return 0;
            const float *x = b ? xs[(b - 1) % 2] : h->x;
            if (!pgpu_head_block(st, &h->mlp[b][0], &h->mlp[b][1], x, B, b ? &prev : NULL,
                                 b ? xs[b % 2] : NULL, h->norm_w[b], h->norm_b[b], 1e-6f,
                                 h->mod + b * ADA, MOD, h->b_mlp[b][0], h->parts[b % 2],
                                 (int)h->cap, h->status))
                return 0;
            prev.parts = h->parts[b % 2];
            prev.gate = h->mod + b * ADA + 2 * PH_WIDTH;
            prev.bias = h->b_mlp[b][1];
        }
        if (cancel && cancel(context))
            return 0;
        return pgpu_head_final(st, &h->final, xs[(HB - 1) % 2], B, &prev, 1e-6f,
                               h->mod + HB * ADA, MOD, h->b_final, lsd ? h->noise : NULL,
                               h->ones, out, out_split, h->eos_rows, EOS_ROWS, eos, h->status);
    }
    for (size_t b = 0; b < HB; b++) {
        if (cancel && cancel(context))
            return 0;
        const float *mod = h->mod + b * ADA;
        if (!pgpu_head_mlp_in(st, &h->mlp[b][0], h->x, B, h->norm_w[b], h->norm_b[b], 1e-6f, mod,
                              MOD, h->b_mlp[b][0], h->first_split, h->status) ||
            !pgpu_gemm_gated(st, &h->mlp[b][1], &first, B, h->b_mlp[b][1], mod + 2 * PH_WIDTH,
                             MOD, h->x, h->x, h->status))
            return 0;
    }
    if (cancel && cancel(context))
        return 0;
    return pgpu_head_final(st, &h->final, h->x, B, NULL, 1e-6f, h->mod + HB * ADA, MOD,
                           h->b_final, lsd ? h->noise : NULL, h->ones, out, out_split,
                           h->eos_rows, EOS_ROWS, eos, h->status);
}

int phonon_flow_head_device_create(const PhononFlowHead *head, const PhononTensorView *eos_weight,
                                   const PhononTensorView *eos_bias, size_t max_streams,
                                   PhononFlowHeadDevice **out) {
    if (!out)
        return 0;
    *out = NULL;
    if (!head || !max_streams || max_streams > 4096 || (!eos_weight) != (!eos_bias) || !ph_init())
        return 0;
    PhononFlowHeadDevice *h = calloc(1, sizeof(*h));
    if (!h)
        return 0;
    h->fused = -1;
    h->one_launch = -1;
    h->use_graph = -1;
    int ok = pgpu_stream_create(&h->own_stream) && (h->stream = h->own_stream) &&
             (h->status = pgpu_malloc(sizeof(int))) &&
             pgpu_memset(h->stream, h->status, 0, sizeof(int)) &&
             upload(h, &head->input_weight, PH_WIDTH, LAT, &h->input) &&
             upload(h, &head->cond_weight, PH_WIDTH, PH_WIDTH, &h->cond) && upload_ada(h, head) &&
             upload(h, &head->final_weight, LAT, PH_WIDTH, &h->final);
    for (size_t b = 0; ok && b < HB; b++)
        for (size_t j = 0; ok && j < 2; j++)
            ok = upload(h, &head->block_mlp_weight[b][j], PH_WIDTH, PH_WIDTH, &h->mlp[b][j]);
    for (size_t i = 0; ok && i < 2; i++)
        ok = upload(h, &head->time_weight[i][0], PH_WIDTH, 256, &h->time_w[i][0]) &&
             upload(h, &head->time_weight[i][1], PH_WIDTH, PH_WIDTH, &h->time_w[i][1]);
    if (ok && eos_weight) {
        h->has_eos = 1;
        ok = upload(h, eos_weight, 1, PH_WIDTH, &h->eos);
    }
    ok = ok && upload_vectors(h, head, eos_bias) && alloc_buffers(h, max_streams) &&
         alloc_flow_buffers(h) &&
         enqueue_tsum(h, 0.0f, 1.0f, h->tsum_lsd) && phonon_flow_head_device_sync(h);
    if (!ok) {
        phonon_flow_head_device_destroy(h);
        return ph_fail("flow head: bad weights or device allocation");
    }
    *out = h;
    return 1;
}

void phonon_flow_head_device_destroy(PhononFlowHeadDevice *h) {
    if (!h)
        return;
    if (h->stream)
        (void)pgpu_stream_sync(h->stream);
    for (size_t i = 0; i < 2; i++)
        pgpu_graph_destroy(h->graphs[i].exec);
    for (size_t i = 0; i < h->nmats; i++)
        pgpu_free(h->mats[i]);
    pgpu_free(h->vec);
    pgpu_free(h->out_norm);
    pgpu_free(h->input_linear_dev);
    pgpu_free(h->buffers);
    pgpu_free(h->flow_buffers);
    pgpu_free(h->tagged_rows);
    pgpu_free(h->tag_word);
    for (size_t i = 0; i < h->nlists; i++)
        pgpu_free(h->lists[i].dev);
    pgpu_free(h->status);
    if (h->own_stream && h->stream != h->own_stream)
        (void)pgpu_stream_sync(h->own_stream);
    pgpu_stream_destroy(h->own_stream);
    free(h);
}

void *phonon_flow_head_device_stream(const PhononFlowHeadDevice *h) {
    return h ? h->stream : NULL;
}

int phonon_flow_head_device_sync(PhononFlowHeadDevice *h) {
    int status = 1;
    if (!h || !pgpu_stream_sync(h->stream) ||
        !pgpu_copy_d2h(h->stream, &status, h->status, sizeof(int)) ||
        !pgpu_memset(h->stream, h->status, 0, sizeof(int)) || !pgpu_stream_sync(h->stream))
        return 0;
    return status == 0;
}

/* The LSD step as one launch (and the counter reset): the same tasks and
 * bits as enqueue_head + the embedding. */
/* The step form for `streams` streams: 0 the chain, 1 one launch, 2 one
 * launch with tagged hand-offs. */
static int lsd_mode(const PhononFlowHeadDevice *h, size_t streams) {
    if (h->one_launch >= 0)
        return h->one_launch;
    return streams <= TAGGED_AUTO_STREAMS ? 2 : 0;
}

static int enqueue_flow(PhononFlowHeadDevice *h, size_t streams, const float *conditions,
                        const float *norm, const float *raw_noise, float scale,
                        float *latents, float *eos_logits, const float *embed, float *next) {
    pgpu_head_flow f;
    memset(&f, 0, sizeof(f));
    f.streams = (int)streams;
    f.tiles = (int)((streams + 15) / 16);
    f.with_eos = eos_logits != NULL;
    f.with_embed = next != NULL;
    f.schedule = flow_list(h, f.tiles, f.with_eos, f.with_embed, &f.tasks);
    if (!f.schedule)
        return ph_fail("flow head: task list");
    f.cond_w = h->cond;
    f.eos_w = h->eos;
    f.ada_w = h->ada;
    f.input_w = h->input;
    f.final_w = h->final;
    f.embed_w = h->input_linear;
    f.conditions = conditions;
    f.out_norm = norm;
    f.b_cond = h->b_cond;
    f.tsum = h->tsum_lsd;
    f.b_eos = h->b_eos;
    f.b_ada = h->b_ada;
    f.b_input = h->b_input;
    f.b_final = h->b_final;
    for (size_t b = 0; b < HB; b++) {
        f.mlp_w[b][0] = h->mlp[b][0];
        f.mlp_w[b][1] = h->mlp[b][1];
        f.b_mlp[b][0] = h->b_mlp[b][0];
        f.b_mlp[b][1] = h->b_mlp[b][1];
        f.norm_w[b] = h->norm_w[b];
        f.norm_b[b] = h->norm_b[b];
    }
    f.raw = raw_noise;
    f.scale = scale;
    f.noise = h->noise;
    f.noise_split = h->noise_split;
    f.silu_split = h->silu_split;
    f.mod = h->mod;
    f.x = h->fx;
    f.u_split = h->fu;
    f.eos_rows = h->eos_rows;
    f.eos = eos_logits;
    f.ones = h->ones;
    f.latents = latents;
    f.latent_split = h->latent_split;
    f.embed_in = embed;
    f.next = next;
    f.counters = h->counters;
    f.status = h->status;
    f.wait_us = h->wait_us;
    f.tagged = lsd_mode(h, streams) == 2;
    if (f.tagged) {
        f.tx = h->tagged_rows;
        f.tu = h->tagged_rows + (size_t)(HB + 1) * h->cap * PH_WIDTH;
        f.tag_word = h->tag_word;
    }
    return pgpu_head_flow_launch(h->stream, &f) &&
           pgpu_head_flow_reset(h->stream, h->counters,
                                (size_t)f.tiles * PGPU_HEADC_KINDS * PGPU_HEAD_COUNTER_STRIDE,
                                f.tagged ? h->tag_word : NULL);
}

/* The tagged words of the one-launch step, cleared, and the tag word set to
 * 1 (allocated on first use). Outside any capture. */
static int reset_tagged(PhononFlowHeadDevice *h) {
    const size_t words = (size_t)(2 * HB + 1) * h->cap * PH_WIDTH;
    if (!h->tagged_rows &&
        !((h->tagged_rows = pgpu_malloc(words * sizeof(uint64_t))) &&
          (h->tag_word = pgpu_malloc(sizeof(unsigned)))))
        return 0;
    const unsigned one = 1;
    if (!pgpu_stream_sync(h->stream) ||
        !pgpu_memset(h->stream, h->tagged_rows, 0, words * sizeof(uint64_t)) ||
        !pgpu_copy_h2d(h->stream, h->tag_word, &one, sizeof(one)) || !pgpu_stream_sync(h->stream))
        return 0;
    h->tag_next = 1;
    return 1;
}

/* The LSD step; with `next` (a frame): the conditions are the decoder's
 * outputs, normalized by out_norm in the head's first launch, and next =
 * input_linear . latents + embed (the latent's embedding; the final launch
 * writes the latent's split fragments into the noise buffer's, which the
 * step no longer reads then). */
static int enqueue_lsd(PhononFlowHeadDevice *h, size_t streams, const float *conditions,
                       const float *raw_noise, float temperature, float *latents,
                       float *eos_logits, const float *embed, float *next) {
    if (lsd_mode(h, streams))
        return enqueue_flow(h, streams, conditions, next ? h->out_norm : NULL, raw_noise,
                            sqrtf(temperature), latents, eos_logits, embed, next);
    if (!enqueue_head(h, streams, conditions, next ? h->out_norm : NULL, raw_noise,
                      sqrtf(temperature), h->tsum_lsd, 1, latents, next ? h->noise_split : NULL,
                      eos_logits, NULL, NULL))
        return 0;
    if (!next)
        return 1;
    const pgpu_gemm_input lat = {.split = h->noise_split};
    return pgpu_gemm_residual(h->stream, &h->input_linear, &lat, (int)streams, embed, next,
                              h->status);
}

/* The step's kernels are captured once per (streams, buffers, temperature)
 * and replayed: two captures are kept, so a caller alternating two sets of
 * buffers replays both. */
static int run_lsd(PhononFlowHeadDevice *h, size_t streams, const float *conditions,
                   const float *raw_noise, float temperature, float *latents, float *eos_logits,
                   const float *embed, float *next) {
    if (!h || !streams || streams > h->cap || !conditions || !raw_noise || !latents ||
        (eos_logits && !h->has_eos) || !(temperature > 0.0f) || !isfinite(temperature))
        return 0;
    /* The kernels move these rows 16 bytes at a time (float4 loads, 64-bit
     * write-through stores): a misaligned pointer is an error, as in the Q8
     * device matvec. */
    const void *aligned[] = {conditions, raw_noise, latents, embed, next};
    for (size_t i = 0; i < sizeof(aligned) / sizeof(aligned[0]); i++)
        if ((uintptr_t)aligned[i] % 16)
            return ph_fail("flow head: device rows must be 16-byte aligned");
    /* The one-launch task list is built (and uploaded) outside any capture. */
    int tasks;
    const int mode = lsd_mode(h, streams);
    if (mode &&
        !flow_list(h, (int)((streams + 15) / 16), eos_logits != NULL, next != NULL, &tasks))
        return ph_fail("flow head: task list");
    /* Every call launches the step once (directly or from its graph), and
     * each launch advances the device tag: the words are allocated on first
     * use and cleared before the tag would wrap. */
    if (mode == 2 && (!h->tagged_rows || h->tag_next >= UINT32_MAX - 1) && !reset_tagged(h))
        return ph_fail("flow head: tagged words");
    if (mode == 2)
        h->tag_next++;
    if (h->use_graph == 0 || (h->use_graph < 0 && mode != 0))
        return enqueue_lsd(h, streams, conditions, raw_noise, temperature, latents, eos_logits,
                           embed, next);
    void *exec = NULL;
    for (size_t i = 0; i < 2 && !exec; i++)
        if (h->graphs[i].exec && h->graphs[i].streams == streams &&
            h->graphs[i].conditions == conditions && h->graphs[i].raw_noise == raw_noise &&
            h->graphs[i].temperature == temperature && h->graphs[i].latents == latents &&
            h->graphs[i].eos_logits == eos_logits && h->graphs[i].embed == embed &&
            h->graphs[i].next == next)
            exec = h->graphs[i].exec;
    if (!exec) {
        const size_t slot = h->graph_victim;
        pgpu_graph_destroy(h->graphs[slot].exec);
        h->graphs[slot].exec = NULL;
        if (!pgpu_graph_begin(h->stream))
            return 0;
        const int enqueued = enqueue_lsd(h, streams, conditions, raw_noise, temperature,
                                         latents, eos_logits, embed, next);
        const int ended = pgpu_graph_end(h->stream, &exec);
        if (!enqueued || !ended) {
            pgpu_graph_destroy(exec);
            return 0;
        }
        h->graphs[slot].exec = exec;
        h->graphs[slot].streams = streams;
        h->graphs[slot].conditions = conditions;
        h->graphs[slot].raw_noise = raw_noise;
        h->graphs[slot].temperature = temperature;
        h->graphs[slot].latents = latents;
        h->graphs[slot].eos_logits = eos_logits;
        h->graphs[slot].embed = embed;
        h->graphs[slot].next = next;
        h->graph_victim = 1 - slot;
    }
    return pgpu_graph_launch(exec, h->stream);
}

int phonon_flow_head_device_lsd(PhononFlowHeadDevice *h, size_t streams,
                                const float *conditions, const float *raw_noise,
                                float temperature, float *latents, float *eos_logits) {
    return run_lsd(h, streams, conditions, raw_noise, temperature, latents, eos_logits, NULL,
                   NULL);
}

int phonon_flow_head_device_set_frame(PhononFlowHeadDevice *h,
                                      const PhononTensorView *out_norm_weight,
                                      const PhononTensorView *out_norm_bias,
                                      const PhononTensorView *input_linear) {
    if (!h || !out_norm_weight || !out_norm_bias || !input_linear || h->has_frame ||
        !pgpu_stream_sync(h->stream))
        return 0;
    float host[2 * PH_WIDTH];
    if (!vec_view(out_norm_weight, PH_WIDTH, host) ||
        !vec_view(out_norm_bias, PH_WIDTH, host + PH_WIDTH))
        return 0;
    float *dev = pgpu_malloc(sizeof(host));
    void *wdev = NULL;
    if (!dev || !pgpu_copy_h2d(h->stream, dev, host, sizeof(host)) ||
        !ph_matrix_upload(input_linear, PH_WIDTH, LAT, &h->input_linear, &wdev) ||
        h->input_linear.q8) {
        pgpu_free(dev);
        pgpu_free(wdev);
        return ph_fail("flow head frame: bad out_norm or input_linear");
    }
    h->out_norm = dev;
    h->input_linear_dev = wdev;
    h->has_frame = 1;
    return 1;
}

int phonon_flow_head_device_frame(PhononFlowHeadDevice *h, size_t streams, const float *outputs,
                                  const float *conditions, const float *raw_noise,
                                  float temperature, float *latents, float *eos_logits,
                                  float *next_inputs) {
    if (!h || !h->has_frame || !conditions || !next_inputs)
        return 0;
    return run_lsd(h, streams, outputs, raw_noise, temperature, latents, eos_logits, conditions,
                   next_inputs);
}

int phonon_flow_head_device_set_stream(PhononFlowHeadDevice *h, void *stream) {
    if (!h || !pgpu_stream_sync(h->stream))
        return 0;
    h->stream = stream ? stream : h->own_stream;
    for (size_t i = 0; i < 2; i++) {
        pgpu_graph_destroy(h->graphs[i].exec);
        h->graphs[i].exec = NULL;
    }
    return 1;
}

int phonon_flow_head_device_set_graph(PhononFlowHeadDevice *h, int use_graph) {
    if (!h)
        return 0;
    if (!pgpu_stream_sync(h->stream))
        return 0;
    if (use_graph < -1 || use_graph > 1)
        return ph_fail("flow head: graph mode must be -1, 0 or 1");
    h->use_graph = use_graph;
    for (size_t i = 0; i < 2; i++) {
        pgpu_graph_destroy(h->graphs[i].exec);
        h->graphs[i].exec = NULL;
    }
    return 1;
}

int phonon_flow_head_device_set_one_launch(PhononFlowHeadDevice *h, int one_launch) {
    if (!h || !pgpu_stream_sync(h->stream))
        return 0;
    if (one_launch < -1 || one_launch > 2)
        return ph_fail("flow head: one-launch mode must be -1, 0, 1 or 2");
    if (one_launch == 2 && !h->tagged_rows && !reset_tagged(h))
        return ph_fail("flow head: tagged words");
    h->one_launch = one_launch;
    for (size_t i = 0; i < 2; i++) {
        pgpu_graph_destroy(h->graphs[i].exec);
        h->graphs[i].exec = NULL;
    }
    return 1;
}

int phonon_flow_head_device_set_fused_mlp(PhononFlowHeadDevice *h, int fused) {
    if (!h || !pgpu_stream_sync(h->stream))
        return 0;
    if (fused < -1 || fused > 1)
        return ph_fail("flow head: fused MLP mode must be -1, 0 or 1");
    h->fused = fused;
    for (size_t i = 0; i < 2; i++) {
        pgpu_graph_destroy(h->graphs[i].exec);
        h->graphs[i].exec = NULL;
    }
    return 1;
}

int phonon_flow_head_device_set_wait_limit(PhononFlowHeadDevice *h, unsigned microseconds) {
    if (!h || !pgpu_stream_sync(h->stream))
        return 0;
    h->wait_us = microseconds;
    for (size_t i = 0; i < 2; i++) {
        pgpu_graph_destroy(h->graphs[i].exec);
        h->graphs[i].exec = NULL;
    }
    return 1;
}

/* ------------------------------------------------ reference-signature API */

enum { REGISTRY = 8 };
static struct {
    const void *key;
    PhononFlowHeadDevice *head;
} registry[REGISTRY];

/* The device copy of `head` (created on first use); call under ph_lock. */
static PhononFlowHeadDevice *lookup(const PhononFlowHead *head, int create) {
    const void *key = head->input_weight.data;
    for (size_t i = 0; i < REGISTRY; i++)
        if (registry[i].key && registry[i].key == key)
            return registry[i].head;
    if (!create)
        return NULL;
    for (size_t i = 0; i < REGISTRY; i++)
        if (!registry[i].key) {
            PhononFlowHeadDevice *h = NULL;
            if (!phonon_flow_head_device_create(head, NULL, NULL, 16, &h))
                return NULL;
            registry[i].key = key;
            registry[i].head = h;
            return h;
        }
    ph_fail("flow head: too many registered heads");
    return NULL;
}

int phonon_flow_head_prepare(const PhononFlowHead *head) {
    if (!head || !head->input_weight.data || !ph_init())
        return 0;
    ph_lock();
    const int ok = lookup(head, 1) != NULL;
    ph_unlock();
    return ok;
}

void phonon_flow_head_release(const PhononFlowHead *head) {
    if (!head)
        return;
    ph_lock();
    for (size_t i = 0; i < REGISTRY; i++)
        if (registry[i].key && registry[i].key == head->input_weight.data) {
            phonon_flow_head_device_destroy(registry[i].head);
            registry[i].key = NULL;
            registry[i].head = NULL;
        }
    ph_unlock();
}

/* One stream through the device head: (s, t) = (0, 1) reuses the cached
 * time embeddings. `raw` is the latent state (lsd = 0) or raw noise scaled
 * by sqrt(temperature) on the device (lsd = 1). */
static int single(const PhononFlowHead *head, const float condition[512], const float raw[32],
                  float s, float t, int lsd, float temperature, float out[32],
                  PhononCancelPoll cancel, void *context) {
    if (!head || !condition || !raw || !out || !isfinite(s) || !isfinite(t) ||
        !ph_all_finite(raw, LAT) || !ph_all_finite(condition, PH_WIDTH) || !ph_init())
        return 0;
    ph_lock();
    PhononFlowHeadDevice *h = lookup(head, 1);
    float result[LAT];
    int ok = h != NULL;
    if (ok) {
        float staged[PH_WIDTH + LAT];
        memcpy(staged, condition, sizeof(float) * PH_WIDTH);
        memcpy(staged + PH_WIDTH, raw, sizeof(float) * LAT);
        const float *cond = h->stage, *state = h->stage + PH_WIDTH;
        const int lsd_times = s == 0.0f && t == 1.0f;
        ok = pgpu_copy_h2d(h->stream, h->stage, staged, sizeof(staged)) &&
             (lsd_times || enqueue_tsum(h, s, t, h->tsum)) &&
             enqueue_head(h, 1, cond, NULL, state, lsd ? sqrtf(temperature) : 1.0f,
                          lsd_times ? h->tsum_lsd : h->tsum, lsd, h->velocity, NULL, NULL, cancel,
                          context) &&
             pgpu_copy_d2h(h->stream, result, h->velocity, sizeof(result)) &&
             phonon_flow_head_device_sync(h);
        if (!ok)
            (void)phonon_flow_head_device_sync(h);  /* drain and clear the record */
    }
    ph_unlock();
    if (!ok || (cancel && cancel(context)))
        return 0;
    memcpy(out, result, sizeof(result));
    return 1;
}

int phonon_flow_head_forward(const PhononFlowHead *head, const float condition[512],
                             const float normalized_state[PHONON_LATENT_WIDTH], float s, float t,
                             float velocity[PHONON_LATENT_WIDTH]) {
    return single(head, condition, normalized_state, s, t, 0, 1.0f, velocity, NULL, NULL);
}

int phonon_flow_lsd_one_step_cancel(const PhononFlowHead *head, const float condition[512],
                                    const float raw_noise[32], float temperature, float output[32],
                                    PhononCancelPoll cancel, void *context) {
    if (!(temperature > 0.0f) || !isfinite(temperature))
        return 0;
    return single(head, condition, raw_noise, 0.0f, 1.0f, 1, temperature, output, cancel,
                  context);
}

int phonon_flow_lsd_one_step(const PhononFlowHead *head, const float condition[512],
                             const float raw_noise[PHONON_LATENT_WIDTH], float temperature,
                             float normalized_latent[PHONON_LATENT_WIDTH]) {
    return phonon_flow_lsd_one_step_cancel(head, condition, raw_noise, temperature,
                                           normalized_latent, NULL, NULL);
}
