/* Internal interfaces of the C17 host layer of libphonon_mi355x. */
#ifndef PH_INTERNAL_H
#define PH_INTERNAL_H

#include "phonon_flow_batch.h"
#include "phonon_gpu.h"
#include "phonon_q8.h"
#include "phonon_transformer.h"

#include <stddef.h>
#include <stdint.h>

enum { PH_WIDTH = 512, PH_HEADS = 8, PH_HEAD = 64, PH_FFN = 2048, PH_SPLIT_KEYS = 256 };
enum { PH_MAX_GROUPS = 4, PH_DEFAULT_GROUPS = 1 };
/* The one-launch step keeps this many positions of headroom in its task
 * schedule (and captured graph) before it has to rebuild them. */
enum { PH_FLOW_HEADROOM = 256 };
/* Batched prefill attention (pgpu_prefill_attention): up to PH_PREFILL_RUN
 * consecutive positions per work entry, fewer while the entries would give
 * under PH_PREFILL_MIN_GROUPS work-groups (one per head per entry). */
enum { PH_PREFILL_RUN = PGPU_PREFILL_RUN, PH_PREFILL_MIN_GROUPS = 1024 };
/* Decode batches of this many 16-stream tiles run as one launch by default
 * (phonon_flow_batch_set_pipeline): measured faster there on MI355X (us per
 * 12-layer step, contexts U{1..2048}, one launch vs phase by phase: B = 1:
 * 349 vs 399; B = 32: 553 vs 648; B = 64: 719 vs 906; B = 128: 1256 vs
 * 1450; B = 192: 1954 vs 2076; B = 224: 2277 vs 2347; B = 256: 2649 vs
 * 2642). */
enum { PH_FLOW_MIN_TILES = 1, PH_FLOW_MAX_TILES = 14 };
/* One-launch steps of at most PH_FLOW_ONE_ROUND_MAX_STREAMS streams, or of
 * PH_FLOW_ONE_ROUND_MIN_TILES..PH_FLOW_ONE_ROUND_MAX_TILES tiles, run one
 * split per ATTN task (the others PGPU_FLOW_ATTN_ROUNDS): us per step, one
 * vs two splits, B = 32: 674 vs 552; B = 48: 693 vs 712; B = 64: 680 vs
 * 689; B = 80: 890 vs 834. */
enum {
    PH_FLOW_ONE_ROUND_MAX_STREAMS = 8,
    PH_FLOW_ONE_ROUND_MIN_TILES = 3,
    PH_FLOW_ONE_ROUND_MAX_TILES = 4
};
/* One-launch steps of at most this many streams hand values over as tagged
 * words (phonon_flow_batch_set_handoff). */
enum { PH_FLOW_TAGGED_MAX_STREAMS = 4 };
/* ... and of at most this many streams skip the MLP-out phase (the fused
 * MLP, PGPU_FLOW_HANDOFF_FUSED_MLP). */
enum { PH_FLOW_FUSED_DEFAULT_MAX_STREAMS = 2 };
/* Chain placement of the one-launch step's task list (pgpu_flow_placement):
 * measured on MI355X at B = 64 (ph_flow_schedule.c). */
pgpu_flow_placement ph_flow_default_placement(int rounds);

/* Device selection and the library's own HIP stream (created once). */
int ph_init(void);
void *ph_stream(void);
/* Serializes the single-stream API (shared scratch and stream). */
void ph_lock(void);
void ph_unlock(void);

/* Records why a call fails (readable through pgpu_last_error) and returns 0;
 * a HIP error already recorded by the failing call is kept. */
int ph_fail(const char *why);

/* Grow-only device scratch owned by the library, for the primitives. */
void *ph_scratch(int slot, size_t bytes);

/* IEEE binary16 -> binary32 (exact) and its finiteness. */
float ph_half_to_float(uint16_t bits);
int ph_half_finite(uint16_t bits);
int ph_bf16_finite(uint16_t bits);
float ph_bf16_to_float(uint16_t bits);

/* Repack a [rows][columns] Q8_0 or BF16 view into MFMA fragment order and
 * upload it, padding rows to 16 and columns to 32 with zeros. `*device`
 * receives the single allocation backing `out` (free with pgpu_free). */
int ph_matrix_upload(const PhononTensorView *view, size_t rows, size_t columns,
                     pgpu_matrix *out, void **device);
/* Decode a BF16 [count] view into `host` (fails on non-finite values). */
int ph_vector_decode(const PhononTensorView *view, size_t count, float *host);

/* (cos, sin) of pair i at `position` for a 64-wide head: fp32 inverse
 * frequency 1/powf(theta, 2i/64) and fp32 phase, as
 * src/phonon_transformer.c:228-233 computes them. */
void ph_rope_row(float theta, size_t position, size_t head_width, float *cos_sin);
/* Device table [8192][32] of (cos, sin) for theta (cached per theta). */
const float *ph_rope_table(float theta);
/* The same for positions [0, PH_ROPE_LONG_ROWS): the Mimi transformer's
 * 16 positions per latent frame, up to 8192 frames. */
enum { PH_ROPE_LONG_ROWS = 8192 * 16 };
const float *ph_rope_table_long(float theta);

int ph_all_finite(const float *values, size_t count);
int ph_overlap(const void *a, size_t a_bytes, const void *b, size_t b_bytes);

/* Enqueue layers [first, first+count) of the step for the batch's active
 * streams, reading the residual stream from `input` and leaving it in
 * `output` (both dev [streams][512]); pool layer = model layer + pool_offset. */
int ph_batch_enqueue_layers(PhononFlowBatch *batch, size_t first, size_t count,
                            size_t pool_offset, const float *input, float *output,
                            float theta);
int ph_batch_set_single(PhononFlowBatch *batch, size_t position, const int32_t *table_dev);
int ph_batch_set_prefill(PhononFlowBatch *batch, size_t streams, const size_t *first,
                         const size_t *counts, const int32_t *tables_dev);
int ph_batch_bind_model(PhononFlowBatch *batch, const PhononFlowModel *model);
float *ph_batch_in(PhononFlowBatch *batch);
float *ph_batch_out(PhononFlowBatch *batch);
size_t ph_batch_table_len(const PhononFlowBatch *batch);
int ph_batch_status(PhononFlowBatch *batch);
const int32_t *ph_batch_tables(const PhononFlowBatch *batch);
float *ph_batch_scratch_rows(PhononFlowBatch *batch);
void *ph_batch_stream(const PhononFlowBatch *batch);
const pgpu_paged_kv *ph_pool_kv(const PhononKvPool *pool);
int *ph_batch_status_word(PhononFlowBatch *batch);
const PhononFlowModel *ph_registered_model(const PhononFlowLayerWeights *weights,
                                           size_t layers);

#endif
