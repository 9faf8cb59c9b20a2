/* Drop-in replacement for the decode-step half of speech-mac
 * src/phonon_transformer.h (src/phonon_transformer.h:1-103). Same types, same
 * signatures, same 1 = success / 0 = failure convention. Every numerical
 * function runs on the MI355X (libphonon_mi355x); host buffers are borrowed
 * and copied to and from device memory inside each call. The pack-side
 * helpers at the end (src/phonon_transformer.h:75-103) read a PhononPack. */
#ifndef PHONON_TRANSFORMER_H
#define PHONON_TRANSFORMER_H

#include "phonon_pack.h"
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/phonon_transformer.h:7-10: request-local cancellation, nonzero stops. A
 * cancelled stack step or prefill resets the cache and publishes nothing. */
typedef int (*PhononCancelPoll)(void *context);
#define PHONON_FLOW_LAYERS 9
#define PHONON_FLOW_WIDTH 512
#define PHONON_FLOW_HEADS 8
#define PHONON_FLOW_HEAD_WIDTH 64

/* src/phonon_transformer.h:16-22. keys/values are the request's host copy in
 * the reference layout [(layer*capacity + position)*512]; the library keeps a
 * device copy of the same rows (paged, block size 16) and writes every row it
 * appends on the device back into keys/values before the call returns. Rows
 * written into keys/values directly by the caller are not seen by the device
 * copy: append through phonon_kv_cache_append. */
typedef struct {
    size_t capacity;
    size_t length;
    float *keys;
    float *values;
} PhononKvCache;

/* src/phonon_transformer.h:24-31. Matrices are Q8_0 or BF16; norm vectors BF16. */
typedef struct {
    const PhononTensorView *qkv;           /* [1536,512], interleaved-RoPE Q/K rows */
    const PhononTensorView *attention_out; /* [512,512] */
    const PhononTensorView *mlp_in;        /* [2048,512] */
    const PhononTensorView *mlp_out;       /* [512,2048] */
    const PhononTensorView *norm1_weight, *norm1_bias;
    const PhononTensorView *norm2_weight, *norm2_bias;
} PhononFlowLayerWeights;

/* src/phonon_transformer.c:16-64. */
int phonon_kv_cache_init(PhononKvCache *cache, size_t capacity);
void phonon_kv_cache_reset(PhononKvCache *cache);
void phonon_kv_cache_destroy(PhononKvCache *cache);
int phonon_kv_cache_append(PhononKvCache *cache, size_t layer, size_t position, const float *key,
                           const float *value, size_t width);
int phonon_kv_cache_commit_position(PhononKvCache *cache, size_t position);

/* Numerical primitives, src/phonon_transformer.c:66-318. */
int phonon_rms_norm(const float *input, const float *weight, size_t width, float epsilon,
                    float *output);
int phonon_layer_norm(const float *input, const float *weight, const float *bias, size_t width,
                      float epsilon, float *output);
int phonon_erf_gelu(float *values, size_t count);
int phonon_rope_interleaved(float *values, size_t width, size_t heads, size_t position,
                            float theta);
int phonon_linear(const PhononTensorView *weight, const float *input, size_t rows, size_t columns,
                  const float *bias, float *output);
int phonon_linear_batch(const PhononTensorView *weight, const float *input, size_t rows,
                        size_t columns, const float *bias, float *output, size_t batch);

/* Decode step, src/phonon_transformer.c:406-489. */
int phonon_flow_layer_step(const PhononFlowLayerWeights *weights, PhononKvCache *cache,
                           size_t layer, size_t position, const float input[PHONON_FLOW_WIDTH],
                           float theta, float output[PHONON_FLOW_WIDTH]);
int phonon_flow_stack_step(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                           PhononKvCache *cache, size_t position,
                           const float input[PHONON_FLOW_WIDTH], float theta,
                           float output[PHONON_FLOW_WIDTH]);
int phonon_flow_stack_step_cancel(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                                  PhononKvCache *cache, size_t position, const float input[512],
                                  float theta, float output[512], PhononCancelPoll cancel,
                                  void *context);
/* src/phonon_transformer.c:619-709. The prefix is run as `length` successive
 * decode steps on the device: mathematically the reference's blocked causal
 * prefill, committed only on success, reset on failure or cancellation. */
int phonon_flow_stack_prefill_cancel(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                                     PhononKvCache *cache, const float *input, size_t length,
                                     float theta, float output[512], PhononCancelPoll cancel,
                                     void *context);
int phonon_flow_stack_prefill(const PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS],
                              PhononKvCache *cache, const float *input, size_t length, float theta,
                              float output[512]);

/* Pack-side helpers, src/phonon_transformer.h:75-103
 * (src/phonon_transformer.c:711-914): voice projection, speaker/duration
 * conditioning, prefix rows, the nine layers' views by checkpoint name,
 * token / BOS / latent embedding into a step input, latent normalization
 * and the decoder's output LayerNorm. */
int phonon_voice_project(const float *voice_latents, size_t frames,
                         const PhononTensorView *projection, float *projected);
int phonon_flow_condition(const PhononTensorView *speaker_embeddings,
                          const PhononTensorView *speaker_projection,
                          const PhononTensorView *duration_projection, size_t speaker_count,
                          float duration_delta, float output[PHONON_FLOW_WIDTH]);
int phonon_flow_prepare_prefix(const int32_t *ids, size_t tokens, const float *token_embeddings,
                               size_t prompt_id, size_t bos_id, const float *projected_voice,
                               size_t voice_frames, const float *bos_latent_projection,
                               float *prefix_embeddings);
int phonon_flow_load_layers(const PhononPack *pack,
                            PhononTensorView storage[PHONON_FLOW_LAYERS][8],
                            PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS]);
int phonon_flow_embed_tokens(const PhononPack *pack, const int32_t *ids, size_t count,
                             float *embeddings);
int phonon_flow_embed_bos(const PhononPack *pack, const float condition[PHONON_FLOW_WIDTH],
                          float output[PHONON_FLOW_WIDTH]);
int phonon_flow_embed_latent(const PhononPack *pack, const float latent[32],
                             const float condition[PHONON_FLOW_WIDTH],
                             float output[PHONON_FLOW_WIDTH]);
int phonon_flow_normalize_latent(const PhononPack *pack, const float denormalized[32],
                                 float normalized[32]);
int phonon_flow_output_norm(const PhononPack *pack, float values[PHONON_FLOW_WIDTH]);

/* Test seam of src/phonon_transformer_test.h:8-9 (phonon_attention_test,
 * src/phonon_transformer.c:578-582): single-query attention of one head over
 * `count` rows of row stride `stride` floats. */
int phonon_attention_test(const float query[64], const float *keys, const float *values,
                          size_t count, size_t stride, float output[64]);

#ifdef __cplusplus
}
#endif

#endif
