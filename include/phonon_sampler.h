/* Flow head of speech-mac's per-frame sampler: the decode output (the
 * condition) and Gaussian noise give the frame's latent in one LSD Euler
 * step; the EOS logit is one more affine row of the condition.
 *
 * The part of src/phonon_sampler.h:11-81 on the per-frame path: the
 * PhononFlowHead view struct and the forward / one-step functions keep the
 * reference's signatures, layouts and 1 = success / 0 = failure convention.
 * (The noise source, stop rules and the generation loop stay in the
 * reference.) The batched device API below it is new: one call advances B
 * streams' frames on the GPU. */
#ifndef PHONON_SAMPLER_H
#define PHONON_SAMPLER_H

#include "phonon_pack.h"
#include "phonon_transformer.h"
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PHONON_LATENT_WIDTH 32
#define PHONON_FLOW_HEAD_BLOCKS 6

/* src/phonon_sampler.h:48-60. Views are borrowed (BF16). */
typedef struct {
    PhononTensorView input_weight, input_bias, cond_weight, cond_bias;
    PhononTensorView time_weight[2][2], time_bias[2][2], time_freqs[2], time_alpha[2];
    PhononTensorView block_ada_weight[PHONON_FLOW_HEAD_BLOCKS];
    PhononTensorView block_ada_bias[PHONON_FLOW_HEAD_BLOCKS];
    PhononTensorView block_norm_weight[PHONON_FLOW_HEAD_BLOCKS];
    PhononTensorView block_norm_bias[PHONON_FLOW_HEAD_BLOCKS];
    PhononTensorView block_mlp_weight[PHONON_FLOW_HEAD_BLOCKS][2];
    PhononTensorView block_mlp_bias[PHONON_FLOW_HEAD_BLOCKS][2];
    PhononTensorView final_ada_weight, final_ada_bias, final_weight, final_bias;
} PhononFlowHead;

/* src/phonon_sampler.h:63 (src/phonon_sampler.c:163-212): every head view
 * from the pack by its checkpoint name (flow_lm.flow_net.*), shapes and
 * BF16 vectors checked; the views are borrowed from the pack. */
int phonon_flow_head_load(const PhononPack *pack, PhononFlowHead *head);
/* src/phonon_sampler.h:64-66: the head's velocity at flow times (s, t) for
 * a normalized latent state. */
int phonon_flow_head_forward(const PhononFlowHead *head, const float condition[512],
                             const float normalized_state[PHONON_LATENT_WIDTH], float s, float t,
                             float velocity[PHONON_LATENT_WIDTH]);
/* src/phonon_sampler.h:68 (src/phonon_sampler.c:395-401): the raw EOS
 * logit flow_lm.out_eos . state + bias (on the device linear). */
int phonon_flow_eos_logit(const PhononPack *pack, const float state[512], float *raw_logit);
/* src/phonon_sampler.h:69-70 (src/phonon_sampler.c:403-418): normalized *
 * flow_lm.emb_std + flow_lm.emb_mean per channel; 0 if a result is not
 * finite. */
int phonon_flow_denormalize_latent(const PhononPack *pack, const float normalized[32],
                                   float denormalized[32]);
/* src/phonon_sampler.h:72-74: noise * sqrt(temperature) plus the velocity at
 * (s, t) = (0, 1). */
int phonon_flow_lsd_one_step(const PhononFlowHead *head, const float condition[512],
                             const float raw_noise[PHONON_LATENT_WIDTH], float temperature,
                             float normalized_latent[PHONON_LATENT_WIDTH]);
/* src/phonon_sampler.h:77-79. The cancel poll runs before each of the six
 * blocks and after the last (as the reference polls); on cancellation
 * returns 0 without publishing output. */
int phonon_flow_lsd_one_step_cancel(const PhononFlowHead *head, const float condition[512],
                                    const float raw_noise[32], float temperature, float output[32],
                                    PhononCancelPoll cancel, void *context);

/* Device copies of heads for the functions above, keyed by the head's
 * input_weight.data: uploaded on first use, or ahead of time here (the
 * analog of phonon_flow_prepare_weights). release frees one. */
int phonon_flow_head_prepare(const PhononFlowHead *head);
void phonon_flow_head_release(const PhononFlowHead *head);

/* -- batched device API (new) -- */
typedef struct PhononFlowHeadDevice PhononFlowHeadDevice;

/* Uploads the head (and, if eos_weight is not NULL, the flow_lm.out_eos row:
 * weight [1][512], bias [1]) for up to max_streams streams per call.
 * Time embeddings of the LSD step (s = 0, t = 1) are computed once, here. */
int phonon_flow_head_device_create(const PhononFlowHead *head, const PhononTensorView *eos_weight,
                                   const PhononTensorView *eos_bias, size_t max_streams,
                                   PhononFlowHeadDevice **out);
void phonon_flow_head_device_destroy(PhononFlowHeadDevice *head);
/* One LSD step of `streams` streams, enqueued on the head's stream: latents
 * = noise * sqrt(temperature) + velocity(condition, noise * sqrt(T); 0, 1)
 * and, if eos_logits is not NULL (and the head has the EOS row), eos_logits[s]
 * = out_eos . condition[s] + bias (src/phonon_sampler.c:395-401). All
 * pointers are device buffers: conditions [streams][512], raw_noise
 * [streams][32], latents [streams][32], eos_logits [streams]. */
int phonon_flow_head_device_lsd(PhononFlowHeadDevice *head, size_t streams,
                                const float *conditions, const float *raw_noise,
                                float temperature, float *latents, float *eos_logits);
/* The pieces of the generation loop around the head, for
 * phonon_flow_head_device_frame (src/phonon_sampler.c:447-483): the
 * decoder's output norm (flow_lm.out_norm weight and bias, BF16 [512];
 * LayerNorm eps 1e-5, src/phonon_transformer.c:904-914) in front of the
 * head, and the latent's embedding (flow_lm.input_linear, BF16 [512][32],
 * no bias, src/phonon_transformer.c:860-874) behind it. Once per head. */
int phonon_flow_head_device_set_frame(PhononFlowHeadDevice *head,
                                      const PhononTensorView *out_norm_weight,
                                      const PhononTensorView *out_norm_bias,
                                      const PhononTensorView *input_linear);
/* One frame of `streams` streams after the decode step (device buffers,
 * 16-byte aligned): state = out_norm(outputs [streams][512]); latents
 * [streams][32] = the LSD step at condition `state`; eos_logits (optional)
 * = out_eos . state + bias; next_inputs [streams][512] = input_linear .
 * latents + conditions [streams][512] (the next decode step's inputs). */
int phonon_flow_head_device_frame(PhononFlowHeadDevice *head, size_t streams,
                                  const float *outputs, const float *conditions,
                                  const float *raw_noise, float temperature, float *latents,
                                  float *eos_logits, float *next_inputs);
/* use_graph = 1: the step's kernels are captured in a HIP graph per
 * (streams, buffers, temperature), two kept, and replayed; 0: each kernel
 * is launched directly; -1 (the default): a graph for the chain of
 * launches, direct launches for the one-launch forms (two kernels: a graph
 * replay costs them 4-5 us at B=1). Returns 0 for any other value. */
int phonon_flow_head_device_set_graph(PhononFlowHeadDevice *head, int use_graph);
/* one_launch = 1: the step runs as one dataflow launch (pgpu_head_flow:
 * every projection a work-group task that waits for its inputs on
 * counters), plus a counter reset; 2: the same launch with the chain's
 * rows (x of each block, its MLP hidden) handed over as tagged words that
 * the consumers poll, no counter between them; 0: the chain of launches;
 * -1 (the default): 2 for steps of at most 2 streams (where it is the
 * fastest form), else 0. All give the same bits. Returns 0 for any other
 * value. */
int phonon_flow_head_device_set_one_launch(PhononFlowHeadDevice *head, int one_launch);
/* fused = 1: the chain runs each residual block as one launch
 * (pgpu_head_block: the MLP-in work-groups also multiply their 64 hidden
 * columns by the MLP-out matrix, and the next launch adds the 8 partials in
 * the MLP-out projection's order), 9 launches per step; 0: two launches per
 * block, 15 per step; -1 (the default): fused for steps of at most 2
 * streams. All give the same bits. Returns 0 for any other value. */
int phonon_flow_head_device_set_fused_mlp(PhononFlowHeadDevice *head, int fused);
/* Bounds a one-launch task's wait for its inputs (microseconds; 0 = 1 s).
 * A wait that gives up ends the launch early and the next sync reports
 * failure. */
int phonon_flow_head_device_set_wait_limit(PhononFlowHeadDevice *head, unsigned microseconds);
/* Runs the head's work on `stream` (a caller's HIP stream, e.g. the decode
 * batch's, so a frame needs no cross-stream hand-off; NULL = the head's
 * own). The caller keeps that stream alive while the head uses it. */
int phonon_flow_head_device_set_stream(PhononFlowHeadDevice *head, void *stream);
/* The head's HIP stream in use (for event timing by the caller). */
void *phonon_flow_head_device_stream(const PhononFlowHeadDevice *head);
/* Waits for enqueued calls; returns 1 iff none saw a non-finite value (and
 * clears that record). */
int phonon_flow_head_device_sync(PhononFlowHeadDevice *head);

#ifdef __cplusplus
}
#endif

#endif
