/* Thin C-ABI layer between the C17 host code and the hand-written gfx950
 * kernels of libphonon_mi355x. Plain pointers and sizes only. Device
 * pointers are marked (dev); `stream` is a HIP stream handle (NULL = the
 * null stream). Functions return 1 on success, 0 on failure, and kernels
 * report non-finite results or invalid indexes by OR-ing a bit into a device
 * status word: 1 = non-finite value, 2 = position/block outside its table.
 *
 * This layer has no counterpart in the reference (a CPU-only C17 program);
 * it is what the drop-in functions of phonon_q8.h / phonon_transformer.h and
 * the batched API of phonon_flow_batch.h are built on. */
#ifndef PHONON_GPU_H
#define PHONON_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A projection matrix resident in device memory in MFMA fragment order.
 * q8 = 1: `values` holds int8 (1 B/weight) and `scales` fp16 bits, one per
 * 32-column block of a row; q8 = 0: `values` holds bf16 and scales is NULL.
 * Fragment order: record (16-row tile t, 32-column block kb) at
 * (t*columns/32 + kb); inside it lane l in 0..63 holds row 16t + l%16,
 * columns 32kb + 8(l/16) .. +7. Scales: [t][kb][16 rows]. */
typedef struct {
    int q8;
    size_t rows, columns;
    const void *values;
    const uint16_t *scales;
} pgpu_matrix;

/* Paged fp32 KV pool: per layer [block][head 8][K|V][16 positions][64]. */
typedef struct {
    float *base;          /* (dev) */
    int layers;
    size_t blocks;        /* blocks per layer */
    size_t layer_stride;  /* floats per layer = blocks * 8 * 2 * 16 * 64 */
} pgpu_paged_kv;

/* Split-attention partials: for (stream s, head h, split j) at slot
 * (s*8 + h)*max_splits + j, the unnormalised P.V row (64 floats) and the
 * split's (max score, sum of exp). */
typedef struct {
    float *part_acc;      /* (dev) [max_streams*8*max_splits][64] */
    float *part_ml;       /* (dev) [max_streams*8*max_splits][2] */
    int max_streams, max_splits;
} pgpu_attention_scratch;

/* The activation operand of a projection, exactly one of:
 *  split     - split fragments (3 bf16 terms per value) of the input rows,
 *              with the stream count rounded up to 16 in the allocation;
 *  rows      - fp32 rows [streams][512], split inside the projection;
 *  ln_rows   - fp32 rows [streams][512], LayerNorm'ed (ln_weight, ln_bias,
 *              ln_epsilon) inside the projection;
 *  attn_acc  - split-attention partials (attn_acc/attn_ml as in
 *              pgpu_attention_scratch, attn_positions and attn_max_splits as
 *              given to pgpu_attention), merged inside the projection.
 * rows, ln_rows and attn_acc need a 512-column matrix. */
typedef struct {
    const uint16_t *split;
    const float *ln_rows, *ln_weight, *ln_bias;
    float ln_epsilon;
    const float *attn_acc, *attn_ml;
    const int32_t *attn_positions;
    int attn_max_splits;
    const float *rows;
} pgpu_gemm_input;

/* -- device, memory, streams, events, graphs (pgpu_runtime.hip) -- */
/* Text of the last failure on this thread (HIP error or failed check). */
const char *pgpu_last_error(void);
void pgpu_record_error(const char *what);
int pgpu_device_init(void);
int pgpu_device_name(char *buffer, size_t size);
void *pgpu_malloc(size_t bytes);
void pgpu_free(void *ptr);
int pgpu_memset(void *stream, void *dst, int value, size_t bytes);
/* Host copies complete before returning. */
int pgpu_copy_h2d(void *stream, void *dst, const void *src, size_t bytes);
/* Pinned host memory (hipHostMalloc), and a host-to-device copy that only
 * enqueues: `src` must be pinned and stay unchanged until the stream has
 * passed the copy. */
void *pgpu_host_malloc(size_t bytes);
void pgpu_host_free(void *ptr);
int pgpu_copy_h2d_async(void *stream, void *dst, const void *src, size_t bytes);
int pgpu_copy_d2h(void *stream, void *dst, const void *src, size_t bytes);
int pgpu_copy_d2d(void *stream, void *dst, const void *src, size_t bytes);
int pgpu_stream_create(void **stream);
void pgpu_stream_destroy(void *stream);
int pgpu_stream_sync(void *stream);
int pgpu_event_create(void **event);
void pgpu_event_destroy(void *event);
int pgpu_event_record(void *event, void *stream);
int pgpu_event_elapsed_ms(void *start, void *stop, float *ms);
/* Work enqueued on `stream` after this call waits for `event`. */
int pgpu_stream_wait_event(void *stream, void *event);
/* Stream capture into a graph: pgpu_graph_begin in thread-local mode;
 * pgpu_graph_begin_global in global mode, where any allocation call made
 * while the capture is open (by any thread) fails the capture. */
int pgpu_graph_begin(void *stream);
int pgpu_graph_begin_global(void *stream);
int pgpu_graph_end(void *stream, void **exec);
int pgpu_graph_launch(void *exec, void *stream);
void pgpu_graph_destroy(void *exec);
int pgpu_check_launch(void);

/* -- projections (pgpu_gemm.hip): out[s][r] = sum_c x[s][c] * W[r][c] -- */
/* out = x.W^T (+ bias), rows of ld_out floats. */
int pgpu_gemm_store(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *x, int streams,
                    const float *bias, float *out, int ld_out, int *status);
/* out = residual + x.W^T, rows of W->rows floats (out may alias residual). */
int pgpu_gemm_residual(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *x,
                       int streams, const float *residual, float *out, int *status);
/* out_split = split fragments of GELU(x.W^T) (the next projection's input). */
int pgpu_gemm_gelu_split(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *x,
                         int streams, uint16_t *out_split, int *status);
/* out_split = split fragments of SiLU((x.W^T + bias) + bias2), bias and
 * bias2 optional [W->rows] vectors (W->rows % 32 == 0). */
int pgpu_gemm_silu_split(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *x,
                         int streams, const float *bias, const float *bias2, uint16_t *out_split,
                         int *status);
/* out = residual + gate * (x.W^T + bias), rows of W->rows floats; gate rows
 * of ld_gate floats, or one gate row for every stream when ld_gate is 0
 * (out may alias residual). */
int pgpu_gemm_gated(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *x, int streams,
                    const float *bias, const float *gate, int ld_gate, const float *residual,
                    float *out, int *status);
/* Fused QKV projection: RoPE on q and k, q scaled by 1/8 into q_out
 * [streams][512], k and v appended to the pool at (layer, positions[s]). */
int pgpu_gemm_qkv(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *x, int streams,
                  const pgpu_paged_kv *kv, int layer, const int32_t *tables, int table_stride,
                  const int32_t *positions, const float *rope, float *q_out, int *status);

/* -- small-batch Q8_0 products on the vector units (pgpu_gemv.hip) --
 * y[s][r] = sum over blocks b of scale[r][b] * (sum_i (float)q[r][32b+i] *
 * x[s][32b+i]) for s < batch <= PGPU_GEMV_MAX_BATCH, with the reference's
 * arithmetic (src/phonon_q8.c:36-62: products rounded, added in column
 * order; blocks added in order), so each output has the bits of
 * phonon_q8_matvec. values: row-major int8 [rows][columns] (16-byte
 * aligned), scales: fp16 bits [rows][columns/32], x [batch][columns]
 * (16-byte aligned), y [batch][rows]; columns = 32 x a divisor of 64. */
#define PGPU_GEMV_MAX_BATCH 8
int pgpu_q8_gemv(void *stream, const int8_t *values, const uint16_t *scales, int rows,
                 int columns, const float *x, int batch, float *y, int *status);

/* -- one-launch decode step (pgpu_flow.hip) --
 * A whole decode step of B streams (all layers) in one launch: every
 * work-group runs one task of the step, named by its descriptor in
 * `schedule`, and first waits for the tasks whose outputs it reads: on
 * counters in device memory, or (tagged mode) by polling the tagged words
 * they write. Tasks, per 16-stream tile t and layer l:
 *   QKV    LayerNorm 1 + QKV projection + RoPE + K/V append, 64 rows each
 *   ATTN   attn_rounds (1..PGPU_FLOW_ATTN_ROUNDS) consecutive 256-key splits
 *          of one (stream, head), one after the other; the task that
 *          completes a (stream, head) merges all its splits
 *   OUT    out projection + residual, 64 rows each
 *   MLP_IN LayerNorm 2 + MLP in projection + GELU, 64 rows each
 *   MLP_OUT MLP out projection + residual, 16 rows each (FUSED_MLP: the last
 *          layer only, its output rows from r and the MLP_IN partials,
 *          64 dimensions each)
 * Descriptor (PGPU_FLOW_TASK) bits: kind [0,3), layer [3,9), tile [9,17),
 * index [17,32); an
 * ATTN index is head | unit << 3 | (stream in tile) << 11, for splits
 * [unit, unit + 1) x attn_rounds. QKV task i computes rows [64i, 64i + 64),
 * i.e. q (i < 8), k (i < 16) or v of head i % 8; an ATTN task of head h
 * waits for QKV tasks h, 8 + h and 16 + h of its tile (of every tile in a
 * batched prefill). A schedule must list every task
 * of the step once, each after every task it depends on (then the launch
 * cannot deadlock); ATTN tasks of (stream, head) must cover the splits of
 * its context. Status bit 4: a wait timed out (1 s), the
 * step's results are then unspecified. */
#define PGPU_FLOW_QKV 0
#define PGPU_FLOW_ATTN 1
#define PGPU_FLOW_OUT 2
#define PGPU_FLOW_MLP_IN 3
#define PGPU_FLOW_MLP_OUT 4
#define PGPU_FLOW_QKV_ALL 5        /* counter only (tile 0): QKV tasks of all tiles */
#define PGPU_FLOW_QKV_HEAD 6       /* counters only, 8 per (layer, tile): the three QKV
                                      tasks of one head (q, k and v rows) */
#define PGPU_FLOW_KINDS 14
#define PGPU_FLOW_QKV_TASKS 24     /* per tile and layer */
#define PGPU_FLOW_OUT_TASKS 8
#define PGPU_FLOW_MLP_IN_TASKS 32
#define PGPU_FLOW_MLP_OUT_TASKS 32
#define PGPU_FLOW_COUNTER_STRIDE 16 /* 32-bit words between phase counters */
#define PGPU_FLOW_ATTN_ROUNDS 2    /* most 256-key splits per ATTN task */
#define PGPU_FLOW_PART_WORDS 72    /* tagged words per split partial (66 used) */
#define PGPU_FLOW_CLEAR_WORDS 2048 /* pgpu_flow_step.clear words zeroed per work-group */
#define PGPU_FLOW_HANDOFF_COUNTER 0 /* pgpu_flow_step.tagged: counters and shared loads */
#define PGPU_FLOW_HANDOFF_TAGGED 1  /* x, r, merged attention rows, split partials tagged */
#define PGPU_FLOW_HANDOFF_PARTS 2   /* split partials tagged, the rest by counters */
#define PGPU_FLOW_HANDOFF_MERGE_OUT 3 /* TAGGED, with no merging attention task: the out
                                       projection merges the split partials itself */
#define PGPU_FLOW_HANDOFF_FUSED_MLP 4 /* MERGE_OUT without an MLP_OUT phase (one tile, decode
                                       only): MLP_IN task i multiplies its 64 GELU rows by
                                       columns [64i, 64i + 64) of the MLP-out matrix,
                                       stores the 512-row partial in `mlp_parts` and counts;
                                       the next layer's QKV tasks wait for the count and add
                                       the PGPU_FLOW_MLP_IN_TASKS partials in task order to
                                       r (QKV tasks 0..7 hand x on to the out projection);
                                       after the last layer PGPU_FLOW_FUSED_OUT_TASKS
                                       MLP_OUT tasks (64 dimensions each) write the output
                                       rows the same way */
#define PGPU_FLOW_FUSED_OUT_TASKS 8
#define PGPU_FLOW_FUSED_MAX_STREAMS 4 /* streams of a FUSED_MLP step */
#define PGPU_FLOW_SCHEDULE_PREFILL 1   /* pgpu_flow_schedule flags */
#define PGPU_FLOW_SCHEDULE_FUSED_MLP 2

#define PGPU_FLOW_TASK(kind, layer, tile, index)                                      \
    ((uint32_t)(kind) | (uint32_t)(layer) << 3 | (uint32_t)(tile) << 9 |             \
     (uint32_t)(index) << 17)

typedef struct {
    const void *values[4];      /* (dev) qkv, out, mlp_in, mlp_out fragments */
    const uint16_t *scales[4];  /* (dev) their Q8 scale planes (NULL: bf16) */
    const float *norms;         /* (dev) [4][512]: norm1 w, b, norm2 w, b */
} pgpu_flow_layer;

typedef struct {
    const pgpu_flow_layer *layers; /* (dev) [layer_count] */
    int layer_count, q8, streams, tiles, prefill;
    int pool_offset;               /* pool layer of model layer 0 */
    const float *input;            /* (dev) [streams][512] layer-0 input */
    float *output;                 /* (dev) [streams][512] last layer's output */
    float *act;                    /* (dev) [layer_count][4][tiles*16][512]: x, r, q, attn */
    uint16_t *hidden;              /* (dev) [layer_count][tiles][64*1536] split fragments */
    float *part_acc;               /* (dev) [layer_count][tiles*16][8][max_splits][64] */
    float *part_ml;                /* (dev) [layer_count][tiles*16][8][ml_group] */
    int max_splits, ml_group;      /* ml_group: floats per (max, sum) group, % 32 == 0 */
    const int32_t *tables, *positions; /* (dev); not written by the step */
    int pos_delta;                 /* stream s is at position positions[s] + pos_delta */
    int table_stride;
    const float *rope;             /* (dev) [8192][32] (cos, sin) */
    const uint32_t *schedule;      /* (dev) one descriptor per work-group */
    unsigned tasks;
    unsigned *phase;               /* (dev) [layer_count][tiles][KINDS] x COUNTER_STRIDE, 0 */
    unsigned *split_done;          /* (dev) [layer_count][tiles*16][8], 0 */
    unsigned *clear;               /* (dev) clear_words words the step sets to 0 (the
                                      counters of the next step), or NULL */
    unsigned clear_words;          /* a multiple of 4, at most PGPU_FLOW_CLEAR_WORDS per
                                      task of the schedule */
    int attn_rounds;               /* 256-key splits per ATTN task, 1..PGPU_FLOW_ATTN_ROUNDS */
    int *status;
    uint64_t *trace;               /* (dev) NULL, or [tasks][4]: start, inputs ready, end
                                      (constant 100 MHz clock) of each task, and where it
                                      ran (XCC id << 32 | HW_ID register) */
    unsigned wait_us;              /* a task's wait for its inputs gives up (status bit 4)
                                      after this many microseconds; 0: one second */
    int tagged;                    /* PGPU_FLOW_HANDOFF_*: TAGGED: x, r, the merged
                                      attention rows and the split partials are handed
                                      over as tagged words in `rows` and `parts`
                                      (part_acc, part_ml and act's x, r and attention
                                      rows are then unused); PARTS: only the split
                                      partials, in `parts` (part_acc, part_ml unused);
                                      MERGE_OUT: as TAGGED, but every attention task
                                      only stores its partials and the out-projection
                                      tasks merge them (no merged attention rows) */
    uint64_t *rows;                /* (dev, TAGGED, MERGE_OUT) [layer_count][6][tiles*16][512]: x, r,
                                      merged attention, and (MERGE_OUT) q, k, v */
    uint64_t *parts;               /* (dev, all but COUNTER) [layer_count][tiles*16][8]
                                      [max_splits][PGPU_FLOW_PART_WORDS]: P.V [64], max,
                                      sum */
    uint32_t tag;                  /* (all but COUNTER) this step's tag, never 0 */
    float *mlp_parts;              /* (dev, FUSED_MLP) [layer_count][PGPU_FLOW_MLP_IN_TASKS]
                                      [16][512]: each MLP_IN task's partial of the MLP-out
                                      projection */
} pgpu_flow_step;

/* Placement of each tile's projection chain in a task list, on a model
 * clock where every attention split task takes unit_us: the tile's OUT,
 * MLP_IN, MLP_OUT and next-layer QKV tasks are listed after_us[0..3] after
 * its last attention task (non-decreasing; a tile's next attention always
 * waits for its QKV). All zero: each chain right behind its attention. */
typedef struct {
    float unit_us;
    float after_us[4];
} pgpu_flow_placement;

/* The task list of a step of `streams` streams through `layers` layers,
 * where stream s lists units[s] ATTN tasks per head (covering its context's
 * splits, plus any headroom: tasks past the live context end at once).
 * Returns the task count; writes the descriptors when `schedule` holds at
 * least that many (`capacity`). Order: QKV of layer 0 for every tile; then
 * for each layer l and tile t, ATTN(t, l) by (stream, split, head) with
 * heads fastest, with the chains OUT, MLP_IN, MLP_OUT (l) and QKV (l+1) of
 * earlier tiles interleaved as `place` (NULL: all zero) sets. Every task
 * follows the tasks it waits for. flags: PGPU_FLOW_SCHEDULE_PREFILL lists
 * all QKV of a layer before its first ATTN (and ignores `place`);
 * PGPU_FLOW_SCHEDULE_FUSED_MLP (decode, one tile) lists no MLP_OUT tasks but
 * the last layer's PGPU_FLOW_FUSED_OUT_TASKS. Host code only. */
size_t pgpu_flow_schedule(size_t streams, size_t layers, const size_t *units,
                          const pgpu_flow_placement *place, int flags, uint32_t *schedule,
                          size_t capacity);
/* prefill = 1: pseudo-streams of one stream share its block table, so an
 * ATTN task waits for the QKV tasks of every tile (one layer-wide count).
 * A step is this one launch: it leaves `positions` as they are (the caller
 * counts the steps in pos_delta) and zeroes `clear` for the next step, so
 * nothing runs between two steps. */
int pgpu_flow_launch(void *stream, const pgpu_flow_step *step, const pgpu_paged_kv *kv);
/* Fills n 32-bit words with `value` (a kernel: usable inside a captured graph). */
int pgpu_fill_u32(void *stream, uint32_t *dst, size_t n, uint32_t value);

/* -- attention (pgpu_attention.hip): stream s attends positions[s]+1 keys;
 * max_splits * 256 must cover every context. Writes the per-split partials
 * into `scratch`; pgpu_attention_merge (or a projection with an attn_acc
 * input) turns them into the attention output. -- */
int pgpu_attention(void *stream, const float *q, const pgpu_paged_kv *kv, int layer,
                   const int32_t *tables, int table_stride, const int32_t *positions,
                   int streams, int heads, int max_splits,
                   const pgpu_attention_scratch *scratch, int *status);
int pgpu_attention_merge(void *stream, const pgpu_attention_scratch *scratch,
                         const int32_t *positions, int streams, int heads, int max_splits,
                         float *out, uint16_t *out_split, int *status);
/* Causal attention of a batched prefill, into the partial layout of
 * pgpu_attention. `entries` (dev) holds entry_count work entries of four
 * int32 (s0, s1, split, unused): streams s0 .. s1-1 (at most 64, all
 * < streams) are consecutive positions of one stream and share the block
 * table row of s0; one work-group per (head, entry) loads keys
 * [256 split, 256 split + 256) of that row once (up to the context of the
 * entry's latest position) and writes split `split`'s partial of every one
 * of those streams whose context reaches it, with pgpu_attention's
 * arithmetic (the same bits). Every split of every stream must be covered by
 * one entry; split < max_splits. */
int pgpu_prefill_attention(void *stream, const float *q, const pgpu_paged_kv *kv, int layer,
                           const int32_t *tables, int table_stride, const int32_t *positions,
                           int streams, int heads, int max_splits, const int32_t *entries,
                           int entry_count, const pgpu_attention_scratch *scratch,
                           int *status);
/* -- audio decoder (pgpu_audio.hip). Positions are rows of row-major
 * [positions][channels] device arrays; every kernel covers all positions of
 * a call at once, taking earlier positions from the caller's history. -- */
/* Mimi input of `frames` latent frames ([frames][32]): the 512 x 32
 * projection (fp32 [512][32]) and the depthwise upsample (fp32 [512][32]:
 * taps 0..15 current frame, 16..31 previous frame) into hidden
 * [16 frames][512]; `previous` (the projection of the frame before, [512])
 * is read for frame 0 and replaced by the last frame's projection. */
int pgpu_mimi_input(void *stream, const float *latents, int frames, const float *projection,
                    const float *upsample, float *previous, float *hidden, int *status);
/* Interleaved RoPE of q (in place) and k of rows [rows][1536] (q | k | v)
 * at positions first + r (rope: [rope_positions][32] (cos, sin) pairs), and
 * k, v stored at ring slot (first + r) % ring of ring_k / ring_v
 * ([ring][512]). */
int pgpu_mimi_rope_store(void *stream, float *qkv, int rows, long long first, const float *rope,
                         long long rope_positions, float *ring_k, float *ring_v, int ring);
/* softmax(q k / 8) v of each row over the keys of positions
 * max(0, p - context + 1) .. p (p = first + r) in the ring, into
 * out [rows][512]; rows a multiple of 16 (whole latent frames), ring >=
 * rows + context - 1 and context <= 256. */
int pgpu_mimi_attention(void *stream, const float *qkv, int rows, long long first,
                        const float *ring_k, const float *ring_v, int ring, int context,
                        float *out, int *status);
/* One SEANet convolution on the device. A causal Conv1d (stride 1, kernel
 * K in {1, 3, 7}) reads taps = K input rows per output row; a causal
 * ConvTranspose1d (stride s in 4..6, kernel 2s) reads taps = 2 (rows t - 1
 * and t) and writes s output positions per input row, as the ncols =
 * s * cout columns (k * cout + o: position t*s + k, channel o) of output
 * row t. Either: `fragments` (cin % 32 == 0): the bf16 weights in MFMA
 * operand order, [P/16][taps*cin/32] records of 64 lanes x 8 bf16, P being
 * ncols rounded up to 32 (lane l of record (i, b): column 16 i + l % 16,
 * zero past ncols, reduction index 32 b + 8 (l / 16) .. +7, index = tap *
 * cin + channel, tap 0 reading row t - taps + 1); or `weight`: fp32
 * [cin][K][cout] for the sequential path. bias [cout]. */
typedef struct {
    int cin, cout, kernel, stride, transpose, taps, ncols;
    const uint16_t *fragments;
    const float *weight;
    const float *bias;
} pgpu_conv_layer;
/* x [positions][cin] -> y [positions][ncols]: y = (residual +) (conv +
 * bias), ELU (x <= 0 ? exp(x) - 1 : x) applied to every input value first
 * when elu is set. Input rows before x come from history [taps-1][cin];
 * history_out (a different buffer) receives the last taps - 1 input rows
 * of [history | x] (unused when taps == 1). With fragments: the MFMA path
 * (bf16 weights times a three-term bf16 split of each input value, fp32
 * accumulation in a fixed order per layer shape); else one fp32 multiply
 * and add per term in the order input channel, then tap (transposed: the
 * current row's sum plus the previous row's). */
int pgpu_conv_rows(void *stream, const pgpu_conv_layer *layer, const float *x, int positions,
                   const float *history, float *history_out, const float *residual, int elu,
                   float *y, int *status);
/* One frame of the depthwise upsample: kernel [channels][2 stride],
 * output[o*channels + c] = previous[c]*k[c][stride+o] + input[c]*k[c][o]. */
int pgpu_upsample_frame(void *stream, const float *kernel, const float *input,
                        const float *previous, int channels, int stride, float *output,
                        int *status);
/* y = x <= 0 ? exp(x) - 1 : x, elementwise (y may be x). */
int pgpu_elu(void *stream, const float *x, float *y, size_t count);

/* -- batched prefill (pgpu_prefill.hip). M = streams pseudo-streams (one per
 * prompt position); split fragments as in pgpu_gemm_input.split, with M
 * rounded up to 16 rows in the allocation. -- */
/* LayerNorm of rows [M][512] (weight, bias, epsilon), into split fragments:
 * the decode step's LayerNorm prologue, the same bits. Only the first
 * `terms` (1..3) split terms of each value are written, or the two fp16
 * terms of PGPU_SPLIT_F16_PAIR. */
int pgpu_rows_split_ln(void *stream, const float *rows, const float *weight, const float *bias,
                       float epsilon, int streams, int terms, uint16_t *out_split, int *status);
/* The split partials of pgpu_attention / pgpu_prefill_attention merged into
 * split fragments with the out-projection prologue's arithmetic (the same
 * bits as a projection with an attn_acc input). */
int pgpu_rows_split_attention(void *stream, const pgpu_attention_scratch *scratch,
                              const int32_t *positions, int streams, int max_splits,
                              uint16_t *out_split, int *status);
/* A projection's weights for the prefill projections: bf16 MFMA fragments
 * in the order of pgpu_matrix values, and for Q8 weights the fp32 block
 * scales [rows/16][columns/32][16] (scales NULL: BF16 weights, no scale)
 * and the same values as fp16 fragments (values_f16, for split terms
 * PGPU_SPLIT_F16_PAIR; NULL: not available). */
typedef struct {
    size_t rows, columns;
    const uint16_t *values;
    const float *scales;
    const uint16_t *values_f16;
} pgpu_wide_matrix;
/* Q8 matrix -> bf16 fragments [rows*columns] and fp32 scales
 * [rows*columns/32] (device buffers): exact conversions. values_f16
 * (optional, NULL: skipped): the int8 values as fp16 fragments (exact). */
int pgpu_wide_from_matrix(void *stream, const pgpu_matrix *w, uint16_t *values, float *scales,
                          uint16_t *values_f16);
/* `terms` value of the split-fragment entry points below: two fp16 terms
 * per activation (hi = fp16(x), lo = fp16(x - hi): 22 significant bits
 * while |x| < 65504; beyond, the outputs are non-finite and flagged) in the
 * records of the first two terms, multiplied on the fp16 matrix cores with
 * the values_f16 weights (two thirds of the three-term work). */
#define PGPU_SPLIT_F16_PAIR 4
/* Projections of M rows of split fragments (K = 512 or 2048; rows a
 * multiple of 128), with the epilogues of pgpu_gemm_qkv, pgpu_gemm_residual
 * and pgpu_gemm_gelu_split. terms = 3: each output has the bits of the
 * single-phase projection of the same weights (the same per-block MFMA
 * sequence, scale order and summation chains); terms = 2: the activations'
 * third split term is left out (each activation taken to 16 significant
 * bits, relative error below 2^-16; two thirds of the matrix-core work);
 * terms = PGPU_SPLIT_F16_PAIR: two fp16 terms with the fp16 weights (22
 * significant bits, two thirds of the work; w->values_f16 required). */
int pgpu_prefill_gemm_qkv(void *stream, const pgpu_wide_matrix *w, const uint16_t *split,
                          int streams, int terms, const pgpu_paged_kv *kv, int layer,
                          const int32_t *tables, int table_stride, const int32_t *positions,
                          const float *rope, float *q_out, int *status);
int pgpu_prefill_gemm_residual(void *stream, const pgpu_wide_matrix *w, const uint16_t *split,
                               int streams, int terms, const float *residual, float *out,
                               int *status);
int pgpu_prefill_gemm_gelu_split(void *stream, const pgpu_wide_matrix *w, const uint16_t *split,
                                 int streams, int terms, uint16_t *out_split, int *status);
/* (The GELU outputs are written as `terms` split terms: the MLP-out
 * projection reads as many. Likewise `terms` of the attention entry points
 * below, 2, 3 or PGPU_SPLIT_F16_PAIR: the split terms of the attention rows
 * written for the out projection.) */
/* Causal attention of a batched prefill, one lane per query, into split
 * fragments of the attention rows (fp32 arithmetic in its own summation
 * order). `runs` (dev) holds run_count pairs (s0, n): pseudo-streams
 * s0 .. s0+n-1 (1 <= n <= PGPU_PREFILL_RUN, all < streams) are consecutive
 * positions of one stream and share the block table row of s0; every
 * pseudo-stream must be in exactly one run. q as written by the QKV
 * projection (scaled by 1/8). Keys [0, position] of each run's stream must
 * be in the pool. */
#define PGPU_PREFILL_RUN 64
int pgpu_prefill_attention_rows(void *stream, const float *q, const pgpu_paged_kv *kv,
                                int layer, const int32_t *tables, int table_stride,
                                const int32_t *positions, int streams, const int32_t *runs,
                                int run_count, uint16_t *out_split, int terms, int *status);
/* The same contract on the matrix cores, over pairs of runs: `pairs` holds
 * (s0, n, s0', n') per pair, two runs of ONE stream (their pseudo-streams
 * share its block-table row; n' = 0: no second run). One work-group per
 * (pair, head) loads each 64-key chunk of the pair's keys once into LDS;
 * waves 0-3 take the first run, 4-7 the second, wave w of a run its queries
 * 16w .. 16w+15; scores, an online softmax per query and the value sums per
 * 16-key sub-block (a query's result does not depend on its pairing).
 * terms 2 or 3: on the fp32 matrix cores (v_mfma_f32_16x16x4_f32, exact
 * fp32 products, sums in the matrix cores' order); PGPU_SPLIT_F16_PAIR: on
 * the fp16 matrix cores, q, K, V and the probabilities each split into two
 * fp16 terms (22 significant bits; products hi.hi + hi.lo + lo.hi; values
 * of magnitude 65520 or more make the output non-finite). Every
 * pseudo-stream must be in exactly one run. */
int pgpu_prefill_attention_mfma(void *stream, const float *q, const pgpu_paged_kv *kv,
                                int layer, const int32_t *tables, int table_stride,
                                const int32_t *positions, int streams, const int32_t *pairs,
                                int pair_count, uint16_t *out_split, int terms, int *status);
/* pgpu_attention followed by pgpu_attention_merge (the same kernels, the
 * same bits), with the split partials in a fixed device-resident array of
 * PGPU_ATTENTION_STATIC_SLOTS (stream, head, split) slots (4.3 MB, held by
 * every GPU the library runs on until the process ends) instead of a
 * caller's pgpu_attention_scratch: the call allocates nothing (no hipMalloc,
 * hipFree or allocating library routine). No counterpart in the reference;
 * for callers that cannot allocate device memory: code under HIP graph
 * capture, serving loops and harnesses that forbid it. Limit: streams * 8 *
 * max_splits <= PGPU_ATTENTION_STATIC_SLOTS (e.g. 64 streams at contexts up
 * to 8192 keys), else it returns 0 with the reason in pgpu_last_error().
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * partials (nothing in it needs clearing: each call writes every partial it
 * reads); calls that overlap in time on one GPU race. */
#define PGPU_ATTENTION_STATIC_SLOTS 16384
int pgpu_attention_static(void *stream, const float *q, const pgpu_paged_kv *kv, int layer,
                          const int32_t *tables, int table_stride, const int32_t *positions,
                          int streams, int heads, int max_splits, float *out,
                          uint16_t *out_split, int *status);

/* -- flow head launches (pgpu_head.hip); BF16 matrices -- */
/* One launch of three independent parts: silu_split = split fragments of
 * SiLU((cond_w . c + cond_bias) + tsum) (tsum optional); if eos_w (16 rows,
 * row 0 live): eos_rows [streams][eos_ld] = eos_w . c + eos_bias; noise =
 * raw * scale ([streams][32], scale positive and finite) and its split
 * fragments (K = 32). c = the rows `conditions`, or their LayerNorm (eps
 * 1e-5) with norm_w and norm_b when those are given. */
int pgpu_head_front(void *stream, const pgpu_matrix *cond_w, const float *conditions, int streams,
                    const float *norm_w, const float *norm_b,
                    const float *cond_bias, const float *tsum, uint16_t *silu_split,
                    const pgpu_matrix *eos_w, const float *eos_bias, float *eos_rows, int eos_ld,
                    const float *raw, float scale, float *noise, uint16_t *noise_split,
                    int *status);
/* One launch: mod [streams][ld_mod] = ada_w . silu + ada_bias and
 * x [streams][512] = input_w . noise + input_bias. */
int pgpu_head_mod(void *stream, const pgpu_matrix *ada_w, const uint16_t *silu_split, int streams,
                  const float *ada_bias, float *mod, int ld_mod, const pgpu_matrix *input_w,
                  const uint16_t *noise_split, const float *input_bias, float *x, int *status);
/* out_split = split fragments of SiLU(w . h + bias), h = LN(x; norm_w, norm_b
 * optional, eps) * (1 + scale) + shift, shift = mod rows [streams][ld_mod],
 * scale 512 columns further. */
int pgpu_head_mlp_in(void *stream, const pgpu_matrix *w, const float *x, int streams,
                     const float *norm_w, const float *norm_b, float eps, const float *mod,
                     int ld_mod, const float *bias, uint16_t *out_split, int *status);
/* A residual block's output handed to the next launch as partials (the
 * fused head chain): x = x_prev + gate * ((P_0 + P_1 + ... + P_7) + bias),
 * the order of pgpu_gemm_gated at K = 512, so x has that launch's bits.
 * P_j = parts + j * ld_parts * 512 ([streams][512] fp32, ld_parts >=
 * streams) is the MLP-out product of hidden columns [64 j, 64 j + 64);
 * gate rows at gate + s * ld_gate; bias [512] (optional). */
typedef struct pgpu_head_parts {
    const float *parts;
    int ld_parts;
    const float *gate;
    int ld_gate;
    const float *bias;
} pgpu_head_parts;
/* A residual block of the head as one launch (the fused chain): x = the
 * rows x, or (prev set) the previous block's output from its partials,
 * whose 512 dimensions are also stored to x_out (required with prev); h =
 * LN(x; norm_w, norm_b, eps) * (1 + scale) + shift (mod rows as
 * pgpu_head_mlp_in); u = SiLU(w_in . h + in_bias); parts_out receives this
 * block's partials of w_out . u (8 of [ld_parts][512], ld_parts >= streams)
 * for the next launch. parts_out and x_out must not overlap x or
 * prev->parts. */
int pgpu_head_block(void *stream, const pgpu_matrix *w_in, const pgpu_matrix *w_out,
                    const float *x, int streams, const pgpu_head_parts *prev, float *x_out,
                    const float *norm_w, const float *norm_b, float eps, const float *mod,
                    int ld_mod, const float *in_bias, float *parts_out, int ld_parts,
                    int *status);
/* out [streams][w->rows] = (residual +) (w . h + bias), h = LN(x; eps) *
 * (1 + scale) + shift as above, x = the rows x or (prev set) the last
 * block's output from its partials; with a residual, `ones` is a [w->rows]
 * vector of 1.0f, and out_split (optional) receives out's split fragments
 * (K = w->rows). If eos: eos[s] = eos_rows[s * eos_ld]. */
int pgpu_head_final(void *stream, const pgpu_matrix *w, const float *x, int streams,
                    const pgpu_head_parts *prev, float eps, const float *mod, int ld_mod,
                    const float *bias, const float *residual, const float *ones, float *out,
                    uint16_t *out_split, const float *eos_rows, int eos_ld, float *eos,
                    int *status);
/* Split fragments (K = 256, stream 0) of [cos | sin](value * freqs[128]). */
int pgpu_head_time_phase(void *stream, const float *freqs, float value, uint16_t *xs,
                         int *status);
/* tsum[512] = 0.5 * (alpha0 * out0 / rms(out0) + alpha1 * out1 / rms(out1)),
 * rms(v) = sqrt(mean(v^2) + 1e-5). */
int pgpu_head_time_sum(void *stream, const float *out0, const float *out1, const float *alpha0,
                       const float *alpha1, float *tsum, int *status);

/* -- the LSD step of the flow head as one launch (pgpu_head.hip) --
 * The projections of pgpu_head_front / _mod / _mlp_in / pgpu_gemm_gated /
 * pgpu_head_final (and, for a frame, the latent embedding) as work-group
 * tasks of one launch, per 16-stream tile t:
 *   COND    8   LN(condition) (or the rows) . cond + b, + tsum, SiLU, split
 *   EOS     1   the EOS row (optional)
 *   NOISE   1   noise = raw * scale, rows and split fragments
 *   INPUT   32  x0 = input . noise + b                   (waits NOISE)
 *   ADA     160 the 10240 modulation rows, 64 per task   (waits COND)
 *   MLP_IN  8   per block b: SiLU(mlp_b0(LN(x_b) * (1 + scale) + shift))
 *               (waits x_b complete and block b's 24 ADA tasks)
 *   MLP_OUT 32  per block b: x_{b+1} = x_b + gate * (mlp_b1 . u + b)
 *   FINAL   1   latent = noise + final(LN(x_6) * (1 + scale) + shift), and
 *               the tile's EOS logits copied out
 *   EMBED   32  next = input_linear . latent + embed (optional)
 * Every task's arithmetic is the chain's, so both give the same bits. A task
 * waits (one lane polls) for per-tile counters; the schedule lists every
 * task after the tasks it waits for, so the launch cannot deadlock. Waits
 * give up after wait_us microseconds (0: 1 s) and set status value 4.
 * Values handed between tasks are stored write-through, each at its own
 * address (x has one buffer per block). The counters must be zero at
 * launch: pgpu_head_flow_reset after each launch. */
enum {
    PGPU_HEAD_COND, PGPU_HEAD_EOS, PGPU_HEAD_NOISE, PGPU_HEAD_INPUT, PGPU_HEAD_ADA,
    PGPU_HEAD_MLP_IN, PGPU_HEAD_MLP_OUT, PGPU_HEAD_FINAL, PGPU_HEAD_EMBED
};
/* Descriptor: kind [0,4), block [4,8), tile [8,16), index [16,32). */
#define PGPU_HEAD_TASK(kind, block, tile, index)                                          \
    ((uint32_t)(kind) | (uint32_t)(block) << 4 | (uint32_t)(tile) << 8 |                  \
     (uint32_t)(index) << 16)
/* Counters per tile (PGPU_HEAD_COUNTER_STRIDE unsigned apart): COND, EOS,
 * NOISE, ADA of blocks 0..6 (6: the final layer's rows), U of blocks 0..5
 * (MLP_IN done), X of versions 0..6, FINAL. */
enum {
    PGPU_HEADC_COND = 0, PGPU_HEADC_EOS = 1, PGPU_HEADC_NOISE = 2, PGPU_HEADC_ADA = 3,
    PGPU_HEADC_U = 10, PGPU_HEADC_X = 16, PGPU_HEADC_FINAL = 23, PGPU_HEADC_KINDS = 24
};
#define PGPU_HEAD_COUNTER_STRIDE 16
#define PGPU_HEAD_BLOCKS 6
typedef struct {
    const uint32_t *schedule; /* (dev) [tasks] */
    int tasks, streams, tiles;
    pgpu_matrix cond_w, eos_w, ada_w, input_w, mlp_w[PGPU_HEAD_BLOCKS][2], final_w, embed_w;
    int with_eos, with_embed;
    const float *conditions;  /* [streams][512] */
    const float *out_norm;    /* [2][512] LayerNorm of the conditions, or NULL */
    const float *b_cond, *tsum, *b_eos, *b_ada, *b_input, *b_mlp[PGPU_HEAD_BLOCKS][2], *b_final;
    const float *norm_w[PGPU_HEAD_BLOCKS], *norm_b[PGPU_HEAD_BLOCKS];
    const float *raw;         /* [streams][32] */
    float scale;
    float *noise;             /* [tiles*16][32] */
    uint16_t *noise_split;    /* split fragments, K = 32 */
    uint16_t *silu_split;     /* K = 512 */
    float *mod;               /* [tiles*16][10240] */
    float *x;                 /* [7][tiles*16][512] */
    uint16_t *u_split;        /* [6] split fragments, K = 512 */
    float *eos_rows;          /* [tiles*16][16] */
    float *eos;               /* [streams] or NULL */
    const float *ones;        /* [32] of 1.0f */
    float *latents;           /* [streams][32] */
    uint16_t *latent_split;   /* K = 32 (embed only) */
    const float *embed_in;    /* [streams][512] (embed only) */
    float *next;              /* [streams][512] (embed only) */
    unsigned *counters;       /* [tiles][PGPU_HEADC_KINDS][PGPU_HEAD_COUNTER_STRIDE], zero */
    int *status;
    unsigned wait_us;
    /* Tagged hand-offs along the chain (tagged != 0): x of versions 0..6 (tx)
     * and SiLU(u) of blocks 0..5 (tu) as 64-bit words, the fp32 value in the
     * low half and the launch's tag in the high half, [7 or 6][tiles*16][512]
     * each; consumers poll the words themselves instead of a producer count.
     * The tag is *tag_word (never 0; pgpu_head_flow_reset advances it). */
    int tagged;
    uint64_t *tx, *tu;
    const unsigned *tag_word;
} pgpu_head_flow;
/* The task list of one launch for `tiles` 16-stream tiles (host code): every
 * task after the tasks it waits for. Writes at most `capacity` descriptors
 * and returns the count (0 if they do not fit; out = NULL only counts). */
int pgpu_head_flow_schedule(uint32_t *out, int capacity, int tiles, int with_eos,
                            int with_embed);
int pgpu_head_flow_launch(void *stream, const pgpu_head_flow *f);
/* Zeroes the launch's counters; with tag_word (optional), also advances the
 * tagged launch's tag (tag_word must not reach 0: its owner clears the
 * tagged words and sets it to 1 before then). */
int pgpu_head_flow_reset(void *stream, unsigned *counters, size_t count, unsigned *tag_word);

/* -- rows and elements (pgpu_elementwise.hip) -- */
int pgpu_ln_split(void *stream, const float *x, int streams, const float *w, const float *b,
                  float eps, uint16_t *xs, float *y, int *status);
int pgpu_split_rows(void *stream, const float *x, int streams, int k_cols, uint16_t *xs,
                    int *status);
int pgpu_norm_row(void *stream, const float *x, int width, const float *w, const float *b,
                  float eps, int rms, float *y, int *status);
int pgpu_gelu(void *stream, float *values, size_t count, int *status);
int pgpu_rope(void *stream, float *values, int heads, int head_width, const float *cos_sin,
              int *status);
/* Copies positions [first_position, first_position+count) of layers
 * [first_layer, first_layer+layers) between the pool (through `table`, dev)
 * and contiguous rows (dev): `keys`/`values` point at the row of
 * (first_layer, first_position); layer y, position x after them lies
 * (y*capacity + x) rows further (the reference [layer][capacity][512] layout
 * when capacity is the cache capacity). */
int pgpu_kv_copy(void *stream, const pgpu_paged_kv *kv, const int32_t *table,
                 int first_position, int count, int first_layer, int layers, float *keys,
                 float *values, size_t capacity, int to_contiguous, int *status);
/* dst[0..count) (count even) = N(0,1) values from `seed` and each pair's
 * index, as pgpu_fill_normal_plan dispatches: it returns their number and,
 * for i below it, the pairs [*first, *first + *pairs) dispatch i fills, at
 * most PGPU_FILL_MAX_GROUPS work-groups of 256 pairs each. */
#define PGPU_FILL_MAX_GROUPS (1u << 23)
size_t pgpu_fill_normal_plan(size_t count, size_t i, size_t *first, size_t *pairs);
int pgpu_fill_normal(void *stream, float *dst, size_t count, uint64_t seed);
/* positions[0..streams) += delta. */
int pgpu_advance_positions(void *stream, int32_t *positions, int streams, int delta);
/* dst[r][0..width) = src[map[r]][0..width) for r < rows (int32 rows; map
 * entries must index rows of src). */
int pgpu_gather_rows(void *stream, int32_t *dst, const int32_t *src, const int32_t *map,
                     int rows, int width);
/* pgpu_gather_rows, and copy_dst[r] = copy_src[r] for r < rows in the same
 * launch (both NULL or both given). A batched prefill gathers its
 * pseudo-streams' block-table rows and copies their positions this way. */
int pgpu_gather_rows_copy(void *stream, int32_t *dst, const int32_t *src, const int32_t *map,
                          int rows, int width, int32_t *copy_dst, const int32_t *copy_src);

#ifdef __cplusplus
}
#endif

#endif
