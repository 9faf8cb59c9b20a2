/* CPU restatement of the speech-mac audio decoder: the Mimi latent
 * transformer (src/phonon_mimi.c), the SEANet convolutions
 * (src/phonon_conv.c) and the latent -> PCM chain (src/phonon_pcm.c).
 * TEST INFRASTRUCTURE ONLY, like the rest of liboracle (see oracle.h).
 * Weights are passed decoded to fp32 (BF16 -> fp32 is exact). The two
 * portable substitutions of oracle.c apply: cblas_sgemm becomes a
 * sequential fp32 dot product per output followed by the alpha/beta update
 * reference BLAS applies, and SLEEF expf4 becomes libm expf. */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { W = 512, CONTEXT = 250, STRIDE = 16, HEADS = 8, HEAD = 64 };

static int finite_all(const float *p, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(p[i]))
            return 0;
    return 1;
}

/* src/phonon_mimi.c:109-131, kernel decoded: [channels][2 stride]. */
int oracle_mimi_upsample_frame(const float *kernel, const float *input, const float *previous,
                               size_t channels, size_t stride, float *output) {
    if (!kernel || !input || !previous || !output || !channels || channels > 512 || !stride ||
        stride > 16)
        return 0;
    for (size_t c = 0; c < channels; c++) {
        if (!isfinite(input[c]) || !isfinite(previous[c]))
            return 0;
        for (size_t o = 0; o < stride; o++) {
            const float current = input[c] * kernel[c * 2 * stride + o];
            const float old = previous[c] * kernel[c * 2 * stride + stride + o];
            output[o * channels + c] = old + current;
            if (!isfinite(output[o * channels + c]))
                return 0;
        }
    }
    return 1;
}

struct OracleMimiState {
    OracleMimi model;
    size_t position;
    float previous[W];
    float keys[2][CONTEXT][W], values[2][CONTEXT][W];
    float hidden[STRIDE][W], normalized[STRIDE][W], qkv[STRIDE][3 * W];
    float attended[STRIDE][W], projected[STRIDE][W], mlp[STRIDE][2048];
    float ordered_keys[CONTEXT][HEAD], ordered_values[CONTEXT][HEAD];
};

OracleMimiState *oracle_mimi_create(const OracleMimi *model) {
    if (!model)
        return NULL;
    OracleMimiState *s = calloc(1, sizeof(*s));
    if (s)
        s->model = *model;
    return s;
}

void oracle_mimi_destroy(OracleMimiState *s) { free(s); }

size_t oracle_mimi_positions(const OracleMimiState *s) { return s ? s->position : 0; }

/* head_order of src/phonon_mimi.c:135-143: even components, then odd. */
static void head_order(const float *in, float *out) {
    for (size_t i = 0; i < 32; i++) {
        out[i] = in[2 * i];
        out[32 + i] = in[2 * i + 1];
    }
}

/* src/phonon_mimi.c:144-199: keys inserted query by query into the 250-slot
 * ring, each query attending min(position + 1, 250) keys. */
static int attention(OracleMimiState *s, size_t layer) {
    float (*ordered_keys)[HEAD] = s->ordered_keys, (*ordered_values)[HEAD] = s->ordered_values;
    for (size_t row = 0; row < STRIDE; row++) {
        const size_t position = s->position + row, slot = position % CONTEXT;
        float *qkv = s->qkv[row];
        if (!oracle_rope_interleaved(qkv, W, HEADS, position, s->model.rope_theta) ||
            !oracle_rope_interleaved(qkv + W, W, HEADS, position, s->model.rope_theta))
            return 0;
        memcpy(s->keys[layer][slot], qkv + W, W * sizeof(float));
        memcpy(s->values[layer][slot], qkv + 2 * W, W * sizeof(float));
        const size_t count = position < CONTEXT - 1 ? position + 1 : CONTEXT;
        const size_t first = position + 1 - count;
        for (size_t h = 0; h < HEADS; h++) {
            float query[HEAD], scores[CONTEXT], dest[HEAD];
            head_order(qkv + h * HEAD, query);
            for (size_t k = 0; k < count; k++) {
                const size_t index = (first + k) % CONTEXT;
                head_order(s->keys[layer][index] + h * HEAD, ordered_keys[k]);
                memcpy(ordered_values[k], s->values[layer][index] + h * HEAD,
                       HEAD * sizeof(float));
            }
            for (size_t k = 0; k < count; k++) {
                float dot = 0.0f;
                for (size_t d = 0; d < HEAD; d++)
                    dot = dot + query[d] * ordered_keys[k][d];
                scores[k] = dot;
            }
            float maximum = -INFINITY;
            for (size_t k = 0; k < count; k++) {
                scores[k] = scores[k] * 0.125f;
                if (!isfinite(scores[k]))
                    return 0;
                if (scores[k] > maximum)
                    maximum = scores[k];
            }
            float lanes[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const size_t end = count - count % 4;
            for (size_t k = 0; k < end; k += 4)
                for (size_t lane = 0; lane < 4; lane++) {
                    scores[k + lane] = expf(scores[k + lane] - maximum);
                    lanes[lane] = lanes[lane] + scores[k + lane];
                }
            float total = (lanes[0] + lanes[2]) + (lanes[1] + lanes[3]);
            for (size_t k = end; k < count; k++) {
                scores[k] = expf(scores[k] - maximum);
                total = total + scores[k];
            }
            if (!(total > 0.0f) || !isfinite(total))
                return 0;
            for (size_t d = 0; d < HEAD; d++) {
                float acc = 0.0f;
                for (size_t k = 0; k < count; k++)
                    acc = acc + scores[k] * ordered_values[k][d];
                dest[d] = acc;
            }
            const float inverse = 1.0f / total;
            for (size_t d = 0; d < HEAD; d++)
                s->attended[row][h * HEAD + d] = dest[d] * inverse;
        }
    }
    return 1;
}

/* src/phonon_mimi.c:200-251. */
static int layer_forward(OracleMimiState *s, size_t l) {
    const OracleMimi *m = &s->model;
    for (size_t row = 0; row < STRIDE; row++)
        if (!oracle_layer_norm(s->hidden[row], m->norm1_weight[l], m->norm1_bias[l], W, 1e-5f,
                               s->normalized[row]))
            return 0;
    for (size_t part = 0; part < 3; part++) {
        if (!oracle_linear_batch(m->qkv[l] + part * W * W, &s->normalized[0][0], W, W, NULL,
                                 &s->projected[0][0], STRIDE))
            return 0;
        for (size_t row = 0; row < STRIDE; row++)
            memcpy(s->qkv[row] + part * W, s->projected[row], W * sizeof(float));
    }
    if (!attention(s, l) ||
        !oracle_linear_batch(m->out[l], &s->attended[0][0], W, W, NULL, &s->projected[0][0],
                             STRIDE))
        return 0;
    for (size_t row = 0; row < STRIDE; row++)
        for (size_t i = 0; i < W; i++)
            s->hidden[row][i] = s->hidden[row][i] + m->scale1[l][i] * s->projected[row][i];
    for (size_t row = 0; row < STRIDE; row++)
        if (!oracle_layer_norm(s->hidden[row], m->norm2_weight[l], m->norm2_bias[l], W, 1e-5f,
                               s->normalized[row]))
            return 0;
    if (!oracle_linear_batch(m->mlp_in[l], &s->normalized[0][0], 2048, W, NULL, &s->mlp[0][0],
                             STRIDE) ||
        !oracle_erf_gelu(&s->mlp[0][0], STRIDE * 2048) ||
        !oracle_linear_batch(m->mlp_out[l], &s->mlp[0][0], W, 2048, NULL, &s->projected[0][0],
                             STRIDE))
        return 0;
    for (size_t row = 0; row < STRIDE; row++)
        for (size_t i = 0; i < W; i++) {
            s->hidden[row][i] = s->hidden[row][i] + m->scale2[l][i] * s->projected[row][i];
            if (!isfinite(s->hidden[row][i]))
                return 0;
        }
    return 1;
}

/* src/phonon_mimi.c:252-283: [frames][32] latents -> [frames*16][512]. */
int oracle_mimi_process(OracleMimiState *s, const float *latents, size_t frames,
                        float *features) {
    if (!s || !latents || !features || !frames || !finite_all(latents, frames * 32))
        return 0;
    for (size_t f = 0; f < frames; f++) {
        float projected[W];
        if (!oracle_linear_batch(s->model.projection, latents + f * 32, W, 32, NULL, projected,
                                 1) ||
            !oracle_mimi_upsample_frame(s->model.upsample, projected, s->previous, W, STRIDE,
                                        &s->hidden[0][0]) ||
            !layer_forward(s, 0) || !layer_forward(s, 1))
            return 0;
        memcpy(s->previous, projected, sizeof(projected));
        memcpy(features + f * STRIDE * W, s->hidden, sizeof(s->hidden));
        s->position += STRIDE;
    }
    return 1;
}

/* ---------------------------------------------------------------- SEANet */
struct OracleConv {
    size_t in, out, kernel, stride;
    int transpose;
    float *weight, *bias, *history, *scratch;
};

OracleConv *oracle_conv_create(const float *weight, const float *bias, size_t in, size_t out,
                               size_t kernel, size_t stride, int transpose) {
    if (!weight || !bias || !in || !out || !kernel || !stride)
        return NULL;
    OracleConv *c = calloc(1, sizeof(*c));
    if (!c)
        return NULL;
    const size_t count = in * out * kernel;
    c->in = in;
    c->out = out;
    c->kernel = kernel;
    c->stride = stride;
    c->transpose = transpose;
    c->weight = malloc(count * sizeof(float));
    c->bias = malloc(out * sizeof(float));
    c->history = calloc(transpose ? out * stride : in * kernel, sizeof(float));
    c->scratch = calloc(transpose ? out * kernel : in * kernel, sizeof(float));
    if (!c->weight || !c->bias || !c->history || !c->scratch) {
        oracle_conv_destroy(c);
        return NULL;
    }
    memcpy(c->weight, weight, count * sizeof(float));
    memcpy(c->bias, bias, out * sizeof(float));
    return c;
}

void oracle_conv_destroy(OracleConv *c) {
    if (!c)
        return;
    free(c->weight);
    free(c->bias);
    free(c->history);
    free(c->scratch);
    free(c);
}

/* src/phonon_conv.c:135-172. Causal Conv1d: weight [out][in][kernel], the
 * history [in][kernel] (im2col order), y = (W . h) + bias. Transposed:
 * weight [in][out][kernel], columns [out][kernel] = W^T x, then
 * y = (column + overlap) + bias for the first `stride` taps and the last
 * `stride` taps kept as the next position's overlap. */
int oracle_conv_process(OracleConv *c, const float *x, size_t n, float *y) {
    if (!c || (n && (!x || !y)) || !finite_all(x, n * c->in))
        return 0;
    for (size_t t = 0; t < n; t++) {
        if (!c->transpose) {
            for (size_t ch = 0; ch < c->in; ch++) {
                float *h = c->history + ch * c->kernel;
                memmove(h, h + 1, (c->kernel - 1) * sizeof(float));
                h[c->kernel - 1] = x[t * c->in + ch];
            }
            const size_t k_count = c->in * c->kernel;
            for (size_t o = 0; o < c->out; o++) {
                float dot = 0.0f;
                for (size_t j = 0; j < k_count; j++)
                    dot = dot + c->weight[o * k_count + j] * c->history[j];
                y[t * c->out + o] = dot + c->bias[o];
            }
        } else {
            const size_t cols = c->out * c->kernel;
            for (size_t j = 0; j < cols; j++) {
                float dot = 0.0f;
                for (size_t ch = 0; ch < c->in; ch++)
                    dot = dot + c->weight[ch * cols + j] * x[t * c->in + ch];
                c->scratch[j] = dot;
            }
            for (size_t k = 0; k < c->stride; k++)
                for (size_t o = 0; o < c->out; o++) {
                    const size_t h = k * c->out + o;
                    y[(t * c->stride + k) * c->out + o] =
                        (c->scratch[o * c->kernel + k] + c->history[h]) + c->bias[o];
                    c->history[h] = c->scratch[o * c->kernel + c->stride + k];
                }
        }
        if (!finite_all(y + t * c->stride * c->out, c->stride * c->out))
            return 0;
    }
    return 1;
}

/* src/phonon_conv.c:173-186: exp(x) - 1 for x <= 0, in place. */
void oracle_conv_elu(float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (x[i] <= 0.0f)
            x[i] = expf(x[i]) - 1.0f;
}

/* src/phonon_conv.c:219-246: y = x + conv1(ELU(conv3(ELU(x)))), one position
 * at a time (conv3: channels -> channels/2, kernel 3; conv1: back, kernel 1). */
int oracle_residual_process(OracleConv *conv3, OracleConv *conv1, const float *x, size_t n,
                            float *y) {
    if (!conv3 || !conv1 || conv3->in != conv1->out || conv3->out != conv1->in)
        return 0;
    float activated[512], hidden[256], result[512];
    const size_t channels = conv3->in, half = conv3->out;
    for (size_t t = 0; t < n; t++) {
        memcpy(activated, x + t * channels, channels * sizeof(float));
        oracle_conv_elu(activated, channels);
        if (!oracle_conv_process(conv3, activated, 1, hidden))
            return 0;
        oracle_conv_elu(hidden, half);
        if (!oracle_conv_process(conv1, hidden, 1, result))
            return 0;
        for (size_t ch = 0; ch < channels; ch++)
            y[t * channels + ch] = x[t * channels + ch] + result[ch];
        if (!finite_all(y + t * channels, channels))
            return 0;
    }
    return 1;
}

/* src/phonon_pcm.c:130-175: per latent frame, Mimi's 16 feature rows, each
 * through conv0, three (ELU, transposed conv, residual) stages of strides
 * 6, 5, 4 and ELU + the final conv: 1920 samples per frame. conv holds
 * conv0, then per stage the transposed conv, conv3 and conv1, then the
 * final conv (the reference's model.conv[] order). */
int oracle_pcm_process(OracleMimiState *mimi, OracleConv *const conv[11], const float *latents,
                       size_t frames, float *pcm) {
    if (!mimi || !conv || !latents || !pcm)
        return 0;
    static const size_t strides[3] = {6, 5, 4};
    float features[STRIDE * W];
    float *a = malloc(120 * 64 * sizeof(float)), *b = malloc(120 * 64 * sizeof(float));
    int ok = a && b;
    for (size_t f = 0; ok && f < frames; f++) {
        ok = oracle_mimi_process(mimi, latents + f * 32, 1, features);
        for (size_t row = 0; ok && row < STRIDE; row++) {
            ok = oracle_conv_process(conv[0], features + row * W, 1, a);
            size_t positions = 1, channels = W;
            for (size_t stage = 0; ok && stage < 3; stage++) {
                oracle_conv_elu(a, positions * channels);
                ok = oracle_conv_process(conv[1 + 3 * stage], a, positions, b);
                positions *= strides[stage];
                channels /= 2;
                ok = ok && oracle_residual_process(conv[2 + 3 * stage], conv[3 + 3 * stage], b,
                                                   positions, a);
            }
            if (ok) {
                oracle_conv_elu(a, positions * channels);
                ok = oracle_conv_process(conv[10], a, 120, pcm + f * 1920 + row * 120);
            }
        }
    }
    free(a);
    free(b);
    return ok;
}
