/* CPU restatement of the speech-mac Flow-transformer decode step.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle of the MI355X
 * product (libphonon_mi355x): only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it. The product never links, calls or
 * falls back to it.
 *
 * Every function follows the arithmetic order of the reference C path
 * (file:line cited per function) with two portable substitutions that the
 * reference's own build cannot avoid off macOS:
 *   - Accelerate cblas_sgemm -> a sequential fp32 dot product per output,
 *     then alpha/beta as reference BLAS applies them;
 *   - SLEEF expf4/sinf4/cosf4 -> the system libm expf/sinf/cosf.
 * Every function is pinned by tests/test_oracle.py: golden vectors from the
 * reference's own tests, the compiled reference phonon_q8.c (oracle/_ref),
 * closed forms, special cases and fp64 restatements. None is unpinned.
 */
#ifndef PHONON_ORACLE_H
#define PHONON_ORACLE_H

#include <stddef.h>
#include <stdint.h>

typedef struct {
    uint16_t scale_bits;
    int8_t values[32];
} OracleQ8Block;

/* One Flow layer with linear weights already expanded to fp32 (row-major
 * [rows][columns]) and norm vectors decoded to fp32. */
typedef struct {
    const float *qkv;     /* [1536][512] */
    const float *out;     /* [512][512] */
    const float *mlp_in;  /* [2048][512] */
    const float *mlp_out; /* [512][2048] */
    const float *norm1_weight, *norm1_bias, *norm2_weight, *norm2_bias; /* [512] each */
} OracleLayer;

float oracle_half_to_float(uint16_t bits);
int oracle_bf16_to_float(const uint16_t *values, size_t count, float *output);
int oracle_q8_dot(const OracleQ8Block *blocks, const float *input, size_t elements,
                  float *result);
int oracle_q8_matvec(const OracleQ8Block *weights, const float *input, size_t rows,
                     size_t columns, float *output);
int oracle_q8_expand(const OracleQ8Block *blocks, size_t rows, size_t columns, float *expanded);
int oracle_linear_batch(const float *expanded, const float *input, size_t rows, size_t columns,
                        const float *bias, float *output, size_t batch);
int oracle_rms_norm(const float *input, const float *weight, size_t width, float epsilon,
                    float *output);
int oracle_layer_norm(const float *input, const float *weight, const float *bias, size_t width,
                      float epsilon, float *output);
int oracle_erf_gelu(float *values, size_t count);
int oracle_rope_interleaved(float *values, size_t width, size_t heads, size_t position,
                            float theta);
int oracle_attention(const float query[64], const float *keys, const float *values, size_t count,
                     size_t stride, float output[64]);
/* Contiguous cache layout of the reference: keys[(layer*capacity+pos)*512 + c]. */
int oracle_kv_append(float *keys, float *values, size_t layers, size_t capacity, size_t layer,
                     size_t position, const float *key, const float *value);
int oracle_layer_step(const OracleLayer *weights, float *keys, float *values, size_t layers,
                      size_t capacity, size_t layer, size_t position, const float input[512],
                      float theta, float output[512]);
int oracle_stack_step(const OracleLayer *weights, size_t layers, float *keys, float *values,
                      size_t capacity, size_t position, const float input[512], float theta,
                      float output[512]);
/* Runs independent streams' stack steps over `threads` pthreads (the CPU
 * baseline for batched decode). Stream s uses keys/values + s*layers*capacity*512
 * and positions[s]; inputs/outputs are [streams][512]. Returns 1 iff all succeed. */
int oracle_stack_step_streams(const OracleLayer *weights, size_t layers, float *keys,
                              float *values, size_t capacity, size_t streams,
                              const size_t *positions, const float *inputs, float theta,
                              float *outputs, size_t threads);

/* Flow head (src/phonon_sampler.h:48-60), linear weights expanded to fp32
 * row-major [rows][columns], vectors decoded to fp32. */
#define ORACLE_HEAD_BLOCKS 6
typedef struct {
    const float *input_weight, *input_bias;               /* [512][32], [512] */
    const float *cond_weight, *cond_bias;                 /* [512][512], [512] */
    const float *time_weight[2][2], *time_bias[2][2];     /* mlp.0 [512][256], mlp.2 [512][512] */
    const float *time_freqs[2], *time_alpha[2];           /* [128], [512] */
    const float *block_ada_weight[ORACLE_HEAD_BLOCKS];    /* [1536][512] */
    const float *block_ada_bias[ORACLE_HEAD_BLOCKS];      /* [1536] */
    const float *block_norm_weight[ORACLE_HEAD_BLOCKS];   /* [512] */
    const float *block_norm_bias[ORACLE_HEAD_BLOCKS];     /* [512] */
    const float *block_mlp_weight[ORACLE_HEAD_BLOCKS][2]; /* [512][512] */
    const float *block_mlp_bias[ORACLE_HEAD_BLOCKS][2];   /* [512] */
    const float *final_ada_weight, *final_ada_bias;       /* [1024][512], [1024] */
    const float *final_weight, *final_bias;               /* [32][512], [32] */
} OracleFlowHead;

float oracle_mean_512(const float input[512]);
int oracle_flow_layer_norm(const float *input, const float *weight, const float *bias,
                           float output[512]);
int oracle_silu(float *values, size_t count);
int oracle_time_embedding(const OracleFlowHead *head, size_t which, float value,
                          float output[512]);
int oracle_flow_head_forward(const OracleFlowHead *head, const float condition[512],
                             const float state[32], float s, float t, float velocity[32]);
int oracle_lsd_one_step(const OracleFlowHead *head, const float condition[512],
                        const float raw_noise[32], float temperature, float output[32]);
/* EOS logit: weight [512] (one row) and bias [1] applied to the state. */
int oracle_eos_logit(const float *weight, const float *bias, const float state[512],
                     float *raw_logit);


/* Audio decoder (oracle_audio.c): Mimi latent transformer, SEANet
 * convolutions and the latent -> PCM chain, weights decoded to fp32. */
typedef struct {
    const float *projection;                 /* [512][32] */
    const float *upsample;                   /* [512][32]: taps 0..15 current, 16..31 previous */
    const float *qkv[2], *out[2];            /* [1536][512], [512][512] */
    const float *mlp_in[2], *mlp_out[2];     /* [2048][512], [512][2048] */
    const float *norm1_weight[2], *norm1_bias[2], *norm2_weight[2], *norm2_bias[2];
    const float *scale1[2], *scale2[2];      /* layer_scale_1 / _2, [512] each */
    float rope_theta;
} OracleMimi;
typedef struct OracleMimiState OracleMimiState;
typedef struct OracleConv OracleConv;
int oracle_mimi_upsample_frame(const float *kernel, const float *input, const float *previous,
                               size_t channels, size_t stride, float *output);
OracleMimiState *oracle_mimi_create(const OracleMimi *model);
void oracle_mimi_destroy(OracleMimiState *state);
size_t oracle_mimi_positions(const OracleMimiState *state);
int oracle_mimi_process(OracleMimiState *state, const float *latents, size_t frames,
                        float *features);
/* weight: Conv1d [out][in][kernel]; transposed [in][out][kernel]. */
OracleConv *oracle_conv_create(const float *weight, const float *bias, size_t in, size_t out,
                               size_t kernel, size_t stride, int transpose);
void oracle_conv_destroy(OracleConv *conv);
int oracle_conv_process(OracleConv *conv, const float *input, size_t positions, float *output);
void oracle_conv_elu(float *values, size_t count);
int oracle_residual_process(OracleConv *conv3, OracleConv *conv1, const float *input,
                            size_t positions, float *output);
int oracle_pcm_process(OracleMimiState *mimi, OracleConv *const conv[11], const float *latents,
                       size_t frames, float *pcm);

#endif
