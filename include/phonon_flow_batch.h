/* Batched decode step for many independent streams on one MI355X.
 *
 * New API with no single counterpart in the reference: speech-mac decodes one
 * request per thread with a contiguous per-request cache (PhononKvCache,
 * src/phonon_transformer.h:16-22). Here B streams advance one position per
 * step through the same L-layer Flow transformer (the math of
 * phonon_flow_stack_step, src/phonon_transformer.c:455-482, per stream),
 * sharing one read of the weights per step, over a paged KV pool with block
 * tables. The single-stream functions of phonon_transformer.h are built on it.
 *
 * Conventions follow the reference: 1 = success, 0 = failure; buffers are
 * borrowed. Objects are not thread-safe: use one batch per thread. */
#ifndef PHONON_FLOW_BATCH_H
#define PHONON_FLOW_BATCH_H

#include "phonon_gpu.h"
#include "phonon_transformer.h"
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PHONON_KV_BLOCK_POSITIONS 16
#define PHONON_FLOW_MAX_POSITIONS 8192

typedef struct PhononFlowModel PhononFlowModel;
typedef struct PhononKvPool PhononKvPool;
typedef struct PhononFlowBatch PhononFlowBatch;

/* Device copy of `layers` layers: the analog of phonon_pack_prepare_linears
 * (src/phonon_pack.c:413-448) for device memory. Q8_0 matrices keep 34 B per
 * 32 weights, repacked into MFMA fragment order; BF16 matrices stay bf16.
 * Fails on a shape, dtype or byte-count mismatch or a non-finite weight. The
 * host views may be released or changed afterwards without effect. */
int phonon_flow_model_create(const PhononFlowLayerWeights *weights, size_t layers,
                             PhononFlowModel **model);
void phonon_flow_model_destroy(PhononFlowModel *model);
size_t phonon_flow_model_layers(const PhononFlowModel *model);
size_t phonon_flow_model_device_bytes(const PhononFlowModel *model);

/* Pool of `blocks` KV blocks; a block holds K and V of 16 positions for all
 * `layers` layers (64 KiB per layer, fp32). Blocks are handed out by id. */
int phonon_kv_pool_create(size_t layers, size_t blocks, PhononKvPool **pool);
void phonon_kv_pool_destroy(PhononKvPool *pool);
size_t phonon_kv_pool_free_blocks(const PhononKvPool *pool);
int phonon_kv_pool_alloc(PhononKvPool *pool, size_t count, int32_t *blocks);
int phonon_kv_pool_release(PhononKvPool *pool, size_t count, const int32_t *blocks);
/* Fills every block with deterministic N(0,1) values (synthetic contexts). */
int phonon_kv_pool_fill_normal(PhononKvPool *pool, uint64_t seed);
/* Copy positions [first, first+count) of all layers between the pool (through
 * `table`, host array of block ids covering those positions) and host arrays
 * in the reference layout keys[(layer*capacity + position)*512]. */
int phonon_kv_pool_write(PhononKvPool *pool, const int32_t *table, size_t table_len,
                         size_t first, size_t count, const float *keys, const float *values,
                         size_t capacity);
int phonon_kv_pool_read(const PhononKvPool *pool, const int32_t *table, size_t table_len,
                        size_t first, size_t count, float *keys, float *values,
                        size_t capacity);
/* The pool's device description, for the kernels of phonon_gpu.h. */
int phonon_kv_pool_view(const PhononKvPool *pool, pgpu_paged_kv *view);

/* A batch of up to max_streams streams of at most max_positions positions
 * (<= 8192) each, bound to a model and a pool with the model's layer count. */
int phonon_flow_batch_create(const PhononFlowModel *model, PhononKvPool *pool,
                             size_t max_streams, size_t max_positions, PhononFlowBatch **batch);
void phonon_flow_batch_destroy(PhononFlowBatch *batch);
/* Sets the active streams: positions[s] is the position stream s decodes
 * next (= its committed length); tables[s*table_len + i] is the pool block
 * of positions [16i, 16i+16), and must cover positions[s] + steps - 1 for
 * every step run before the next call. */
int phonon_flow_batch_set_streams(PhononFlowBatch *batch, size_t streams,
                                  const size_t *positions, const int32_t *tables,
                                  size_t table_len);
/* One decode step of every active stream: inputs/outputs host [streams][512].
 * Appends one K/V row per layer at each stream's position, then advances the
 * positions. Returns 0 (positions still advanced, outputs unspecified) if
 * any value is non-finite or a position is not covered by its table. */
int phonon_flow_batch_step(PhononFlowBatch *batch, const float *inputs, float theta,
                           float *outputs);
/* The same step with device-resident inputs/outputs [streams][512] (dev),
 * enqueued on the batch's stream without waiting. The step is captured into a
 * HIP graph on first use and replayed afterwards. */
int phonon_flow_batch_step_device(PhononFlowBatch *batch, const float *inputs, float theta,
                                  float *outputs);
/* Batched prefill (the batched form of phonon_flow_stack_prefill,
 * src/phonon_transformer.c:622-702, for many streams and chunks): positions
 * [first[i], first[i] + counts[i]) of stream i, whose block table is row i of
 * `tables` (host [streams][table_len]), all run through the model's layers in
 * one pass. inputs/outputs (dev) hold one [512] row per position, stream by
 * stream in position order; each output row is what a decode step at that
 * position returns. Positions below first[i] must already be in the pool.
 * Uses the batch's stream slots (sum of counts <= max_streams): call
 * phonon_flow_batch_set_streams before the next phonon_flow_batch_step*.
 * Enqueued without waiting; phonon_flow_batch_sync reports non-finite values. */
int phonon_flow_batch_prefill_device(PhononFlowBatch *batch, size_t streams, const size_t *first,
                                     const size_t *counts, const int32_t *tables,
                                     size_t table_len, const float *inputs, float theta,
                                     float *outputs);
/* Arithmetic of phase-by-phase batched prefills: 1 exact: the projections
 * with the decode step's three bf16 split terms and the decode step's split
 * attention and merge, so every output row has the bits of single steps;
 * 0 (default) and 2 fast: where a layer's matrices are Q8, the projections
 * on the fp16 matrix cores with two fp16 split terms of each activation (22
 * significant bits), and a causal attention that loads each 64-key chunk
 * once per run of 64 positions: 0 on the fp16 matrix cores with the same
 * two-term splits of q, K, V and the probabilities, 2 with one lane per
 * query on the vector units (fp32). The fast modes stay within 1e-4 of the
 * exact one (normwise per row). */
int phonon_flow_batch_set_prefill_exact(PhononFlowBatch *batch, int exact);
/* One-launch step: a task that has waited this many microseconds for its
 * inputs (at most 10 s) gives up, sets status bit 2 (value 4) and makes
 * every other waiting task give up, so the launch ends; its results are
 * then unusable (phonon_flow_batch_sync returns 0). 0 (the default): one
 * second. A small value forces that path from the host. */
int phonon_flow_batch_set_wait_limit(PhononFlowBatch *batch, unsigned microseconds);
/* Runs the streams as `groups` (1..4) independent groups of whole 16-stream
 * tiles, each on its own HIP stream inside the step's graph. Results do not
 * depend on it. Default 1: on MI355X under ROCm 7 kernels of different HIP
 * streams were measured not to overlap, so more groups only add launches. */
int phonon_flow_batch_set_groups(PhononFlowBatch *batch, size_t groups);
/* mode 2: each step (and batched prefill) is one launch holding every
 * layer's work as a dataflow graph of work-group tasks (pgpu_flow_launch):
 * one 16-stream tile's projections run while other tiles' attention
 * streams K/V, and no launch boundary separates the phases. mode 0: one
 * launch per phase of each layer. mode 1 (default): one launch for the
 * decode batch sizes where that measured faster on MI355X (1..224 streams),
 * phase by phase otherwise. Results are identical (both run the same task
 * code). Batches over 4096 streams, models over 63 layers and models mixing
 * Q8 and BF16 matrices always run phase by phase. */
int phonon_flow_batch_set_pipeline(PhononFlowBatch *batch, int mode);
/* Placement of the projection chains in the one-launch step's task list
 * (pgpu_flow_placement); NULL restores the default. Results do not depend
 * on it. */
int phonon_flow_batch_set_placement(PhononFlowBatch *batch, const pgpu_flow_placement *place);
/* Task timeline of the one-launch step: while set, every step whose task
 * list fits `capacity` tasks writes, for task i, trace[4i .. 4i+2] = start,
 * inputs ready, end on the GPU's constant 100 MHz clock and trace[4i+3] =
 * where it ran (XCC id << 32 | HW_ID register) (trace: dev, 4 * capacity
 * words). NULL, 0 turns it off. */
int phonon_flow_batch_set_trace(PhononFlowBatch *batch, uint64_t *trace, size_t capacity);
/* The one-launch step's current task list (pgpu_flow_schedule order):
 * returns the task count, and copies it when capacity suffices; 0 before the
 * first one-launch step. */
size_t phonon_flow_batch_schedule(const PhononFlowBatch *batch, uint32_t *schedule,
                                  size_t capacity);
/* One-launch step: 256-key attention splits per ATTN task (1 or 2; 0, the
 * default: chosen by the batch size). Results are identical for every
 * choice. */
int phonon_flow_batch_set_attention_rounds(PhononFlowBatch *batch, int rounds);
/* One-launch step: how tasks hand the layer output, the out projection,
 * the merged attention rows and the split partials to each other: 1 as
 * tagged words the consumer polls (one memory round trip less per hand-off,
 * for a few streams); 0 through counters and shared cacheable loads; 2 the
 * split partials as tagged words, the rest through counters (an attention
 * task then need not wait for its partial to reach memory); 3 as 1, but
 * the out-projection tasks merge the split partials themselves (no
 * attention task waits to merge); 4 as 3, with no MLP-out phase: each
 * MLP-in task multiplies its GELU rows by its columns of the MLP-out matrix
 * and the next layer's QKV tasks add the 32 partials (batches of at most 4
 * streams; larger batches run mode 3); -1 (the default) by the batch size.
 * Modes 0-3 give identical results; mode 4 sums the MLP-out products in
 * another order (within fp32 rounding of the others). */
int phonon_flow_batch_set_handoff(PhononFlowBatch *batch, int tagged);
/* Kernel timing: while `before` and `after` are events (pgpu_event_create),
 * each step launches its kernels directly (no graph replay) and records
 * `before` right before and `after` right after its one-launch kernel
 * (k_flow_step, the whole step) on the batch's stream. Phase-by-phase steps
 * record nothing. NULL, NULL turns it off. */
int phonon_flow_batch_set_timing(PhononFlowBatch *batch, void *before, void *after);
/* use_graph = 1 (default): a phase-by-phase step_device replays a captured
 * HIP graph (a one-launch step is always launched directly: one kernel
 * gains nothing from a graph); 0: it launches the step's kernels directly
 * (e.g. for a caller that is itself capturing a graph). Results are
 * identical. */
int phonon_flow_batch_set_graph(PhononFlowBatch *batch, int use_graph);
/* Waits for enqueued steps; returns 1 iff no step since the last call saw a
 * non-finite value or an uncovered position (and clears that record). */
int phonon_flow_batch_sync(PhononFlowBatch *batch);
/* The step status word since the last phonon_flow_batch_sync, without
 * clearing it: bit 0 non-finite value, 1 position/block outside its table,
 * 2 (value 4) a one-launch wait timed out. Waits for enqueued steps. */
int phonon_flow_batch_status(PhononFlowBatch *batch, int *status);
/* Current positions (host mirror) of the active streams. */
int phonon_flow_batch_positions(const PhononFlowBatch *batch, size_t *positions);
/* The batch's HIP stream (for event timing by the caller). */
void *phonon_flow_batch_stream(const PhononFlowBatch *batch);
/* Device buffers of [max_streams][512] fp32 owned by the batch, convenient
 * as step_device inputs/outputs. */
float *phonon_flow_batch_device_inputs(PhononFlowBatch *batch);
float *phonon_flow_batch_device_outputs(PhononFlowBatch *batch);

/* Registers a device copy of weights[0..layers) for the single-stream
 * functions of phonon_transformer.h: later calls with this same array (same
 * view pointers) use it instead of uploading per call. Like the reference's
 * prepared materializations, the registered weights must not change. */
int phonon_flow_prepare_weights(const PhononFlowLayerWeights *weights, size_t layers);
void phonon_flow_release_weights(const PhononFlowLayerWeights *weights);

#ifdef __cplusplus
}
#endif

#endif
