/* Drop-in replacement for speech-mac src/phonon_mimi.h:1-47: the Mimi latent
 * transformer (latent frame -> 16 feature rows). Same types, signatures and
 * 1 = success / 0 = failure convention. A state keeps its weights (bf16 MFMA
 * fragments), its rotary K/V ring and its scratch on the MI355X; a call runs
 * every frame of the request through each layer at once (all 16 x frames
 * positions in one pass per layer, causal over a 250-key window), host
 * buffers being copied in and out inside the call. */
#ifndef PHONON_MIMI_H
#define PHONON_MIMI_H

#include "phonon_transformer.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PHONON_MIMI_WIDTH 512
#define PHONON_MIMI_CONTEXT 250
#define PHONON_MIMI_STRIDE 16
#define PHONON_MIMI_MAX_FRAMES 8192

/* src/phonon_mimi.h:10-16. */
typedef struct {
    unsigned sample_rate;
    float frame_rate;
    unsigned ratios[3];
    size_t context;
    float rope_theta;
} PhononMimiConfig;
/* src/phonon_mimi.h:17-24: borrowed pack views (projection [512,32,1],
 * upsample [512,1,32], per layer in_proj, out_proj, linear1, linear2,
 * norm1 w/b, norm2 w/b, layer_scale_1, layer_scale_2). The views must
 * outlive the model; a state copies what it needs to the device. */
typedef struct {
    PhononMimiConfig config;
    size_t stride;
    PhononTensorView projection, upsample;
    PhononTensorView layers[2][10];
} PhononMimiModel;
typedef struct PhononMimiState PhononMimiState;

/* src/phonon_mimi.h:27-36. */
PhononMimiConfig phonon_mimi_config(void);
int phonon_mimi_model_load(const PhononPack *pack, const PhononMimiConfig *config,
                           PhononMimiModel *model);
int phonon_mimi_state_create(const PhononMimiModel *model, PhononMimiState **state);
void phonon_mimi_state_reset(PhononMimiState *state);
void phonon_mimi_state_destroy(PhononMimiState *state);
size_t phonon_mimi_positions(const PhononMimiState *state);
/* src/phonon_mimi.h:37-42: row-major [frames,32] -> [frames*16,512]; capacity
 * in feature rows; input and output must not overlap. On a processing
 * failure the state is unusable until reset (the output may hold a partial
 * prefix); invalid arguments leave it untouched. At most 8192 frames per
 * request. */
int phonon_mimi_process(PhononMimiState *state, const float *latents, size_t frames,
                        float *features, size_t capacity);
/* src/phonon_mimi.h:43-46: depthwise causal transposed convolution of one
 * frame ([channels, 2*stride] kernel, no bias, right trim of stride):
 * output[offset*channels + c] = previous[c]*k[c][stride+offset] +
 * input[c]*k[c][offset]. */
int phonon_mimi_upsample_frame(const PhononTensorView *weight, const float *input,
                               const float *previous, size_t channels, size_t stride,
                               float *output);

#ifdef __cplusplus
}
#endif
#endif
