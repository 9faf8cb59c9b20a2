/* Drop-in replacement for speech-mac src/phonon_conv.h:1-45: the dense SEANet
 * operators (causal Conv1d, stride 1, kernel 1/3/7; causal ConvTranspose1d,
 * stride 4/5/6, kernel 2*stride; channels 1..512) and the residual seam.
 * A model keeps its weights (fp32) on the MI355X; a state keeps its history
 * there. A call computes all of its positions at once (each output position
 * reads the input window it needs, the previous call's tail coming from the
 * state), host buffers being copied in and out inside the call. */
#ifndef PHONON_CONV_H
#define PHONON_CONV_H

#include "phonon_pack.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct PhononConvModel PhononConvModel;
typedef struct PhononConvState PhononConvState;
/* src/phonon_conv.h:11-18. weight: Conv1d [out,in,kernel], transposed
 * [in,out,kernel], BF16; bias [out] BF16. */
int phonon_conv_model_create(const PhononTensorView *weight, const PhononTensorView *bias,
                             size_t stride, int transpose, PhononConvModel **model);
void phonon_conv_model_destroy(PhononConvModel *model);
size_t phonon_conv_input_channels(const PhononConvModel *model);
size_t phonon_conv_output_channels(const PhononConvModel *model);
size_t phonon_conv_stride(const PhononConvModel *model);
/* src/phonon_conv.h:19-31: row-major [positions,channels]; capacity counts
 * output positions; each input position emits `stride` outputs at once; at
 * most 15,728,640 cumulative input positions; zero positions is a no-op;
 * invalid arguments leave the state unchanged; an arithmetic failure
 * poisons it until reset. Buffers must not overlap. */
int phonon_conv_state_create(const PhononConvModel *model, PhononConvState **state);
void phonon_conv_state_destroy(PhononConvState *state);
void phonon_conv_state_reset(PhononConvState *state);
int phonon_conv_process(PhononConvState *state, const float *input, size_t positions,
                        float *output, size_t capacity);
/* src/phonon_conv.h:33-36: in place, x <= 0 -> exp(x) - 1 (host buffer). */
void phonon_conv_elu(float *values, size_t count);
/* src/phonon_conv.h:38-44: identity + Conv1(ELU(Conv3(ELU(input)))), hidden
 * width channels/2; the models must outlive the state. */
typedef struct PhononResidualState PhononResidualState;
int phonon_residual_state_create(const PhononConvModel *conv3, const PhononConvModel *conv1,
                                 PhononResidualState **state);
void phonon_residual_state_destroy(PhononResidualState *state);
void phonon_residual_state_reset(PhononResidualState *state);
int phonon_residual_process(PhononResidualState *state, const float *input, size_t positions,
                            float *output, size_t capacity);

#ifdef __cplusplus
}
#endif
#endif
