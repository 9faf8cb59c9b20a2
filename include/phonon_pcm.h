/* Drop-in replacement for speech-mac src/phonon_pcm.h:1-37: denormalized
 * latent frames -> mono 24 kHz PCM through Mimi and the SEANet decoder. The
 * chain runs on the MI355X: a call takes every frame of the request through
 * Mimi in one pass per layer, then through each SEANet stage at once (16,
 * 96, 480 and 1920 positions per frame), keeping every intermediate in
 * device memory; host buffers are copied in and out inside the call. */
#ifndef PHONON_PCM_H
#define PHONON_PCM_H

#include "phonon_conv.h"
#include "phonon_mimi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PHONON_PCM_FRAME_SAMPLES 1920
#define PHONON_PCM_SAMPLE_RATE 24000

typedef struct PhononPCMModel PhononPCMModel;
typedef struct PhononPCMState PhononPCMState;
/* src/phonon_pcm.h:10-19. */
int phonon_pcm_model_create(const PhononPack *pack, PhononPCMModel **model);
void phonon_pcm_model_destroy(PhononPCMModel *model);
int phonon_pcm_state_create(const PhononPCMModel *model, PhononPCMState **state);
void phonon_pcm_state_destroy(PhononPCMState *state);
void phonon_pcm_state_reset(PhononPCMState *state);
size_t phonon_pcm_samples(const PhononPCMState *state);
/* src/phonon_pcm.h:20-32: [frames,32] -> frames*1920 samples into raw (and
 * final, which may be NULL or raw, else must not overlap); capacities count
 * samples; at most 8192 frames per request. */
int phonon_pcm_process(PhononPCMState *state, const float *latents, size_t frames, float *raw,
                       size_t raw_capacity, float *final, size_t final_capacity);
/* src/phonon_pcm.h:33-36. */
int phonon_pcm_finish(PhononPCMState *state);

/* Test seam (the role of src/phonon_pcm_test.h:6-8): a PCM model from a Mimi
 * model's views and eleven convolution models in the reference's order
 * (conv0; per stride 6, 5, 4 the transposed conv, conv3, conv1; the final
 * conv). Takes ownership of the convolution models on success. */
int phonon_pcm_model_from_parts(const PhononMimiModel *mimi, PhononConvModel *conv[11],
                                PhononPCMModel **model);

#ifdef __cplusplus
}
#endif
#endif
