/* CPU restatement of the speech-mac decode step. TEST INFRASTRUCTURE ONLY:
 * see oracle.h for who may load it and which leaf operations are portable
 * substitutes. Built with -std=c17 -O2 -ffp-contract=off so no multiply-add
 * is contracted unless the reference writes fmaf explicitly. */
#include "oracle.h"

#include <limits.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

enum { WIDTH = 512, HEADS = 8, HEAD = 64, FFN = 2048, MAX_POSITIONS = 8192 };

static float bits_to_float(uint32_t bits) {
    float value;
    memcpy(&value, &bits, sizeof(value));
    return value;
}

/* IEEE binary16 -> binary32, exact for every pattern.
 * Follows src/phonon_q8.c:7-34 (duplicate at src/phonon_pack.c:343-370). */
float oracle_half_to_float(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits >> 15) << 31;
    uint32_t exponent = (bits >> 10) & 31u, fraction = bits & 1023u;
    if (exponent == 31u)
        return bits_to_float(sign | 0x7f800000u | (fraction << 13));
    if (exponent != 0u)
        return bits_to_float(sign | ((exponent + 112u) << 23) | (fraction << 13));
    if (fraction == 0u)
        return bits_to_float(sign);
    /* Subnormal: shift the leading one into the implicit position. */
    uint32_t e = 113u;
    while (!(fraction & 1024u)) {
        fraction <<= 1;
        e--;
    }
    return bits_to_float(sign | (e << 23) | ((fraction & 1023u) << 13));
}

/* src/phonon_pack.c:321-341: bf16 bits are the high half of a binary32. */
int oracle_bf16_to_float(const uint16_t *values, size_t count, float *output) {
    if (!values || !output || !count)
        return 0;
    for (size_t i = 0; i < count; i++) {
        float v = bits_to_float((uint32_t)values[i] << 16);
        if (!isfinite(v))
            return 0;
        output[i] = v;
    }
    return 1;
}

/* src/phonon_q8.c:36-62: per block, serial fp32 partial of q*x, then
 * sum += scale*partial. Non-finite scale, input or sum fails. */
int oracle_q8_dot(const OracleQ8Block *blocks, const float *input, size_t elements,
                  float *result) {
    if (!blocks || !input || !result || !elements || elements % 32)
        return 0;
    float sum = 0.0f;
    for (size_t b = 0; b < elements / 32; b++) {
        const float scale = oracle_half_to_float(blocks[b].scale_bits);
        if (!isfinite(scale))
            return 0;
        const float *x = input + b * 32;
        float partial = 0.0f;
        for (size_t i = 0; i < 32; i++) {
            if (!isfinite(x[i]))
                return 0;
            const float product = (float)blocks[b].values[i] * x[i];
            partial = partial + product;
        }
        const float scaled = scale * partial;
        sum = sum + scaled;
    }
    if (!isfinite(sum))
        return 0;
    *result = sum;
    return 1;
}

static int ranges_overlap(const void *a, size_t a_bytes, const void *b, size_t b_bytes) {
    uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + b_bytes && y < x + a_bytes;
}

/* src/phonon_q8.c:64-92: row-wise dot; input/output and weights/output must
 * not overlap. */
int oracle_q8_matvec(const OracleQ8Block *weights, const float *input, size_t rows,
                     size_t columns, float *output) {
    if (!weights || !input || !output || !rows || !columns || columns % 32 ||
        rows > SIZE_MAX / (columns / 32) / sizeof(OracleQ8Block))
        return 0;
    const size_t per_row = columns / 32;
    if (ranges_overlap(input, columns * sizeof(float), output, rows * sizeof(float)) ||
        ranges_overlap(weights, rows * per_row * sizeof(OracleQ8Block), output,
                       rows * sizeof(float)))
        return 0;
    for (size_t r = 0; r < rows; r++)
        if (!oracle_q8_dot(weights + r * per_row, input, columns, output + r))
            return 0;
    return 1;
}

/* src/phonon_pack.c:396-407: each weight expands to scale*(float)q before any
 * projection (exact in fp32: an 11-bit by 8-bit product). */
int oracle_q8_expand(const OracleQ8Block *blocks, size_t rows, size_t columns, float *expanded) {
    if (!blocks || !expanded || !rows || !columns || columns % 32)
        return 0;
    for (size_t b = 0; b < rows * columns / 32; b++) {
        const float scale = oracle_half_to_float(blocks[b].scale_bits);
        if (!isfinite(scale))
            return 0;
        for (size_t i = 0; i < 32; i++)
            expanded[b * 32 + i] = scale * (float)blocks[b].values[i];
    }
    return 1;
}

/* Portable stand-in for cblas_sgemm(RowMajor, NoTrans, Trans, M, N, K, 1, A, K,
 * B, K, beta, C, N): each C[m][n] = (serial fp32 sum over k) + beta*C[m][n]. */
static void sgemm_nt(size_t m_count, size_t n_count, size_t k_count, const float *a,
                     size_t lda, const float *b, size_t ldb, float beta, float *c, size_t ldc) {
    for (size_t m = 0; m < m_count; m++)
        for (size_t n = 0; n < n_count; n++) {
            float acc = 0.0f;
            for (size_t k = 0; k < k_count; k++) {
                const float product = a[m * lda + k] * b[n * ldb + k];
                acc = acc + product;
            }
            c[m * ldc + n] = beta == 0.0f ? acc : acc + beta * c[m * ldc + n];
        }
}

/* Portable stand-in for cblas_sgemm(RowMajor, NoTrans, NoTrans, 1, N, K, 1,
 * a, K, B, ldb, beta, c, N): c[n] = (serial sum over k of a[k]*B[k][n]) + beta*c[n]. */
static void sgemv_t(size_t n_count, size_t k_count, const float *a, const float *b, size_t ldb,
                    float beta, float *c) {
    for (size_t n = 0; n < n_count; n++) {
        float acc = 0.0f;
        for (size_t k = 0; k < k_count; k++) {
            const float product = a[k] * b[k * ldb + n];
            acc = acc + product;
        }
        c[n] = beta == 0.0f ? acc : acc + beta * c[n];
    }
}

/* src/phonon_transformer.c:253-313: outputs start at bias (or 0), then one
 * SGEMM with beta = bias ? 1 : 0; every input and output must be finite. */
int oracle_linear_batch(const float *expanded, const float *input, size_t rows, size_t columns,
                        const float *bias, float *output, size_t batch) {
    if (!expanded || !input || !output || !rows || !columns || !batch)
        return 0;
    for (size_t i = 0; i < batch * columns; i++)
        if (!isfinite(input[i]))
            return 0;
    for (size_t r = 0; r < batch * rows; r++) {
        if (bias && !isfinite(bias[r % rows]))
            return 0;
        output[r] = bias ? bias[r % rows] : 0.0f;
    }
    for (size_t i = 0; i < rows * columns; i++)
        if (!isfinite(expanded[i]))
            return 0;
    sgemm_nt(batch, rows, columns, input, columns, expanded, columns, bias ? 1.0f : 0.0f, output,
             rows);
    for (size_t r = 0; r < batch * rows; r++)
        if (!isfinite(output[r]))
            return 0;
    return 1;
}

/* src/phonon_transformer.c:66-85. */
int oracle_rms_norm(const float *input, const float *weight, size_t width, float epsilon,
                    float *output) {
    if (!input || !weight || !output || !width || !(epsilon > 0.0f) || !isfinite(epsilon))
        return 0;
    double squares = 0.0;
    for (size_t i = 0; i < width; i++) {
        if (!isfinite(input[i]) || !isfinite(weight[i]))
            return 0;
        squares += (double)input[i] * input[i];
    }
    const float scale = 1.0f / sqrtf((float)(squares / (double)width) + epsilon);
    if (!isfinite(scale))
        return 0;
    for (size_t i = 0; i < width; i++) {
        output[i] = input[i] * scale * weight[i];
        if (!isfinite(output[i]))
            return 0;
    }
    return 1;
}

/* Welford merge of a group (count add, mean a1, M2 a2) into a running
 * (n, m1, m2), unfused: src/phonon_transformer.c:90-98. */
static void welford_merge(size_t add, float a1, float a2, size_t *n, float *m1, float *m2) {
    const size_t total = *n + add;
    const float c = total ? (float)add / (float)total : 0.0f;
    const float delta = a1 - *m1;
    const float step = c * delta;
    *m1 = *m1 + step;
    const float d2 = delta * delta;
    const float d2c = d2 * c;
    const float d2cn = d2c * (float)*n;
    const float grow = a2 + d2cn;
    *m2 = *m2 + grow;
    *n = total;
}

/* Mean and population variance of 512 floats in the reference's order:
 * 8 chunks of 16 four-lane Welford updates, a three-level cascade of chunk
 * merges, a flush of the cascade into level 0, and a scalar four-lane merge
 * whose mean update and M2 growth use fmaf as written in the reference.
 * src/phonon_transformer.c:99-151. */
static void moments_of_512(const float *x, float *mean, float *variance) {
    float level_m1[3][4] = {{0}}, level_m2[3][4] = {{0}};
    size_t level_n[3] = {0};
    for (size_t chunk = 0; chunk < 8; chunk++) {
        float m1[4] = {0}, m2[4] = {0};
        for (size_t j = 0; j < 16; j++)
            for (size_t lane = 0; lane < 4; lane++) {
                const float v = x[chunk * 64 + j * 4 + lane];
                const float delta = v - m1[lane];
                const float inv = 1.0f / (float)(j + 1);
                const float step = delta * inv;
                m1[lane] = m1[lane] + step;
                const float after = v - m1[lane];
                const float grow = delta * after;
                m2[lane] = m2[lane] + grow;
            }
        for (size_t lane = 0; lane < 4; lane++) {
            size_t n = level_n[0];
            welford_merge(16, m1[lane], m2[lane], &n, &level_m1[0][lane], &level_m2[0][lane]);
        }
        level_n[0] += 16;
        /* Carry full levels upward like a binary counter over chunks. */
        size_t bits = chunk + 1;
        for (size_t level = 1; level < 3 && !(bits & 1u); level++, bits >>= 1) {
            for (size_t lane = 0; lane < 4; lane++) {
                size_t n = level_n[level];
                welford_merge(level_n[level - 1], level_m1[level - 1][lane],
                              level_m2[level - 1][lane], &n, &level_m1[level][lane],
                              &level_m2[level][lane]);
                level_m1[level - 1][lane] = 0.0f;
                level_m2[level - 1][lane] = 0.0f;
            }
            level_n[level] += level_n[level - 1];
            level_n[level - 1] = 0;
        }
    }
    for (size_t level = 1; level < 3; level++) {
        for (size_t lane = 0; lane < 4; lane++) {
            size_t n = level_n[0];
            welford_merge(level_n[level], level_m1[level][lane], level_m2[level][lane], &n,
                          &level_m1[0][lane], &level_m2[0][lane]);
        }
        level_n[0] += level_n[level];
    }
    float m1 = 0.0f, m2 = 0.0f;
    size_t n = 0;
    for (size_t lane = 0; lane < 4; lane++) {
        const size_t total = n + 128;
        const float c = 128.0f / (float)total;
        const float delta = level_m1[0][lane] - m1;
        m1 = fmaf(c, delta, m1);
        const float d2 = delta * delta;
        const float d2c = d2 * c;
        m2 = m2 + fmaf(d2c, (float)n, level_m2[0][lane]);
        n = total;
    }
    *mean = m1;
    *variance = m2 / 512.0f;
}

/* src/phonon_transformer.c:153-185: width 512 uses the Welford moments;
 * other widths use double two-pass moments. y = ((x-mean)*rstd)*w + b. */
int oracle_layer_norm(const float *input, const float *weight, const float *bias, size_t width,
                      float epsilon, float *output) {
    if (!input || !weight || !bias || !output || !width || !(epsilon > 0.0f) ||
        !isfinite(epsilon))
        return 0;
    double sum = 0.0;
    for (size_t i = 0; i < width; i++) {
        if (!isfinite(input[i]) || !isfinite(weight[i]) || !isfinite(bias[i]))
            return 0;
        sum += input[i];
    }
    double mean = sum / (double)width;
    float variance;
    if (width == 512) {
        float m, v;
        moments_of_512(input, &m, &v);
        mean = m;
        variance = v;
    } else {
        double squares = 0.0;
        for (size_t i = 0; i < width; i++) {
            const double centered = (double)input[i] - mean;
            squares += centered * centered;
        }
        variance = (float)(squares / (double)width);
    }
    const float scale = 1.0f / sqrtf(variance + epsilon);
    for (size_t i = 0; i < width; i++) {
        const float centered = (float)((double)input[i] - mean);
        const float normalized = centered * scale;
        const float weighted = normalized * weight[i];
        output[i] = weighted + bias[i];
        if (!isfinite(output[i]))
            return 0;
    }
    return 1;
}

/* Abramowitz & Stegun 7.1.26 erf with the fmaf chain of the reference's
 * Torch-NEON adaptation: src/phonon_transformer.c:190-200. */
static float erf_as7126(float x) {
    const float t = 1.0f / fmaf(0.3275911f, fabsf(x), 1.0f);
    float r = fmaf(1.061405429f, t, -1.453152027f);
    r = fmaf(r, t, 1.421413741f);
    r = fmaf(r, t, -0.284496736f);
    r = fmaf(r, t, 0.254829592f);
    const float square = x * x;
    const float neg_exp = -expf(-square);
    const float tn = t * neg_exp;
    return copysignf(fmaf(tn, r, 1.0f), x);
}

/* src/phonon_transformer.c:202-216: full four-element groups use the
 * polynomial erf, the count%4 tail uses libm erff. */
int oracle_erf_gelu(float *values, size_t count) {
    if (!values && count)
        return 0;
    const size_t groups_end = count - count % 4;
    for (size_t i = 0; i < count; i++) {
        if (!isfinite(values[i]))
            return 0;
        const float scaled = values[i] * 0.7071067811865475244f;
        const float e = i < groups_end ? erf_as7126(scaled) : erff(scaled);
        const float half = 0.5f * values[i];
        const float one_plus = 1.0f + e;
        values[i] = half * one_plus;
        if (!isfinite(values[i]))
            return 0;
    }
    return 1;
}

/* src/phonon_transformer.c:218-251: fp32 inverse frequency 1/powf(theta,
 * 2i/head), fp32 phase pos*freq, rotation of interleaved pairs (2i, 2i+1)
 * of every head, unfused. cos/sin from libm (the reference uses SLEEF u10
 * for full groups of four). */
int oracle_rope_interleaved(float *values, size_t width, size_t heads, size_t position,
                            float theta) {
    if (!values || !width || !heads || width % heads || (width / heads) % 2 ||
        !(theta > 0.0f) || !isfinite(theta))
        return 0;
    const size_t head = width / heads;
    for (size_t i = 0; i < head / 2; i++) {
        const float exponent = (float)(2 * i) / (float)head;
        const float freq = 1.0f / powf(theta, exponent);
        const float phase = (float)position * freq;
        const float c = cosf(phase), s = sinf(phase);
        for (size_t h = 0; h < heads; h++) {
            float *pair = values + h * head + 2 * i;
            const float a = pair[0], b = pair[1];
            if (!isfinite(a) || !isfinite(b) || !isfinite(c) || !isfinite(s))
                return 0;
            const float ac = a * c, bs = b * s, as = a * s, bc = b * c;
            pair[0] = ac - bs;
            pair[1] = as + bc;
            if (!isfinite(pair[0]) || !isfinite(pair[1]))
                return 0;
        }
    }
    return 1;
}

/* Copy `rows` head vectors (row stride `stride`) into [rows][64] with the
 * even components first, then the odd ones: src/phonon_transformer.c:330-336. */
static void even_odd_order(const float *input, size_t rows, size_t stride, float *output) {
    for (size_t r = 0; r < rows; r++)
        for (size_t i = 0; i < 32; i++) {
            output[r * 64 + i] = input[r * stride + 2 * i];
            output[r * 64 + 32 + i] = input[r * stride + 2 * i + 1];
        }
}

/* Single-query causal attention over `count` keys with 512-key online-softmax
 * blocks: src/phonon_transformer.c:338-404. */
int oracle_attention(const float query[64], const float *keys, const float *values, size_t count,
                     size_t stride, float output[64]) {
    if (!query || !keys || !values || !output || !count || count > MAX_POSITIONS ||
        stride < 64 || stride > INT_MAX)
        return 0;
    float running_max = -INFINITY, total = 0.0f, dest[64] = {0};
    float q[64];
    float *k_block = malloc(512 * 64 * sizeof(float));
    float *scores = malloc(512 * sizeof(float));
    if (!k_block || !scores) {
        free(k_block);
        free(scores);
        return 0;
    }
    int ok = 0;
    even_odd_order(query, 1, 64, q);
    for (size_t start = 0; start < count; start += 512) {
        const size_t length = count - start < 512 ? count - start : 512;
        even_odd_order(keys + start * stride, length, stride, k_block);
        sgemm_nt(1, length, 64, q, 64, k_block, 64, 0.0f, scores, length);
        float block_max = running_max;
        for (size_t i = 0; i < length; i++) {
            scores[i] = scores[i] * 0.125f;
            if (!isfinite(scores[i]))
                goto done;
            if (scores[i] > block_max)
                block_max = scores[i];
        }
        /* Four-lane sums over full groups, reduced (0+2)+(1+3), then a
         * serial tail. */
        float lanes[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const size_t groups_end = length - length % 4;
        for (size_t i = 0; i < groups_end; i += 4)
            for (size_t lane = 0; lane < 4; lane++) {
                scores[i + lane] = expf(scores[i + lane] - block_max);
                lanes[lane] = lanes[lane] + scores[i + lane];
            }
        float block_sum = (lanes[0] + lanes[2]) + (lanes[1] + lanes[3]);
        for (size_t i = groups_end; i < length; i++) {
            scores[i] = expf(scores[i] - block_max);
            block_sum = block_sum + scores[i];
        }
        const float rescale = expf(running_max - block_max);
        total = fmaf(rescale, total, block_sum);
        running_max = block_max;
        if (start)
            for (size_t d = 0; d < 64; d++)
                dest[d] = dest[d] * rescale;
        /* Both the K=1 legacy branch and the portable GEMV compute a rounded
         * product sum followed by a separate add of the prior value. */
        sgemv_t(64, length, scores, values + start * stride, stride, start ? 1.0f : 0.0f, dest);
    }
    if (!(total > 0.0f) || !isfinite(total))
        goto done;
    const float inverse = 1.0f / total;
    for (size_t d = 0; d < 64; d++) {
        output[d] = dest[d] * inverse;
        if (!isfinite(output[d]))
            goto done;
    }
    ok = 1;
done:
    free(k_block);
    free(scores);
    return ok;
}

/* src/phonon_transformer.c:45-57 with the layer count as a parameter. */
int oracle_kv_append(float *keys, float *values, size_t layers, size_t capacity, size_t layer,
                     size_t position, const float *key, const float *value) {
    if (!keys || !values || !key || !value || layer >= layers || position >= capacity)
        return 0;
    for (size_t i = 0; i < WIDTH; i++)
        if (!isfinite(key[i]) || !isfinite(value[i]))
            return 0;
    const size_t offset = (layer * capacity + position) * WIDTH;
    memcpy(keys + offset, key, WIDTH * sizeof(float));
    memcpy(values + offset, value, WIDTH * sizeof(float));
    return 1;
}

/* src/phonon_transformer.c:406-453 (layer count as a parameter). */
int oracle_layer_step(const OracleLayer *w, float *keys, float *values, size_t layers,
                      size_t capacity, size_t layer, size_t position, const float input[512],
                      float theta, float output[512]) {
    if (!w || !keys || !values || !input || !output || layer >= layers ||
        position >= capacity || position >= MAX_POSITIONS)
        return 0;
    float normalized[WIDTH], residual[WIDTH], projected[3 * WIDTH], attended[WIDTH];
    float attention[WIDTH], *mlp = malloc(FFN * sizeof(float));
    if (!mlp)
        return 0;
    int ok = 0;
    if (!oracle_layer_norm(input, w->norm1_weight, w->norm1_bias, WIDTH, 1e-5f, normalized) ||
        !oracle_linear_batch(w->qkv, normalized, 3 * WIDTH, WIDTH, NULL, projected, 1))
        goto done;
    float *q = projected, *k = projected + WIDTH, *v = projected + 2 * WIDTH;
    if (!oracle_rope_interleaved(q, WIDTH, HEADS, position, theta) ||
        !oracle_rope_interleaved(k, WIDTH, HEADS, position, theta) ||
        !oracle_kv_append(keys, values, layers, capacity, layer, position, k, v))
        goto done;
    for (size_t h = 0; h < HEADS; h++) {
        const size_t offset = layer * capacity * WIDTH + h * HEAD;
        if (!oracle_attention(q + h * HEAD, keys + offset, values + offset, position + 1, WIDTH,
                              attended + h * HEAD))
            goto done;
    }
    if (!oracle_linear_batch(w->out, attended, WIDTH, WIDTH, NULL, attention, 1))
        goto done;
    for (size_t i = 0; i < WIDTH; i++)
        residual[i] = input[i] + attention[i];
    if (!oracle_layer_norm(residual, w->norm2_weight, w->norm2_bias, WIDTH, 1e-5f, normalized) ||
        !oracle_linear_batch(w->mlp_in, normalized, FFN, WIDTH, NULL, mlp, 1) ||
        !oracle_erf_gelu(mlp, FFN) ||
        !oracle_linear_batch(w->mlp_out, mlp, WIDTH, FFN, NULL, output, 1))
        goto done;
    for (size_t i = 0; i < WIDTH; i++) {
        output[i] = output[i] + residual[i];
        if (!isfinite(output[i]))
            goto done;
    }
    ok = 1;
done:
    free(mlp);
    return ok;
}

/* src/phonon_transformer.c:455-482 without cancellation or the length
 * bookkeeping (the caller owns positions). */
int oracle_stack_step(const OracleLayer *weights, size_t layers, float *keys, float *values,
                      size_t capacity, size_t position, const float input[512], float theta,
                      float output[512]) {
    if (!weights || !layers || !input || !output || position >= capacity)
        return 0;
    float a[WIDTH], b[WIDTH];
    memcpy(a, input, sizeof(a));
    for (size_t layer = 0; layer < layers; layer++) {
        if (!oracle_layer_step(&weights[layer], keys, values, layers, capacity, layer, position,
                               a, theta, b))
            return 0;
        memcpy(a, b, sizeof(a));
    }
    memcpy(output, a, sizeof(a));
    return 1;
}

typedef struct {
    const OracleLayer *weights;
    size_t layers, capacity, first, last;
    float *keys, *values;
    const size_t *positions;
    const float *inputs;
    float *outputs;
    float theta;
    int ok;
} StreamJob;

static void *run_streams(void *arg) {
    StreamJob *job = arg;
    const size_t per_stream = job->layers * job->capacity * WIDTH;
    job->ok = 1;
    for (size_t s = job->first; s < job->last; s++)
        if (!oracle_stack_step(job->weights, job->layers, job->keys + s * per_stream,
                               job->values + s * per_stream, job->capacity, job->positions[s],
                               job->inputs + s * WIDTH, job->theta, job->outputs + s * WIDTH))
            job->ok = 0;
    return NULL;
}

int oracle_stack_step_streams(const OracleLayer *weights, size_t layers, float *keys,
                              float *values, size_t capacity, size_t streams,
                              const size_t *positions, const float *inputs, float theta,
                              float *outputs, size_t threads) {
    if (!weights || !keys || !values || !positions || !inputs || !outputs || !streams ||
        !threads)
        return 0;
    if (threads > streams)
        threads = streams;
    StreamJob *jobs = calloc(threads, sizeof(StreamJob));
    pthread_t *ids = calloc(threads, sizeof(pthread_t));
    if (!jobs || !ids) {
        free(jobs);
        free(ids);
        return 0;
    }
    int ok = 1;
    size_t started = 0;
    for (size_t t = 0; t < threads; t++) {
        jobs[t] = (StreamJob){weights, layers, capacity, streams * t / threads,
                              streams * (t + 1) / threads, keys, values, positions, inputs,
                              outputs, theta, 0};
        if (pthread_create(&ids[t], NULL, run_streams, &jobs[t]) != 0) {
            ok = 0;
            break;
        }
        started++;
    }
    for (size_t t = 0; t < started; t++) {
        pthread_join(ids[t], NULL);
        ok &= jobs[t].ok;
    }
    free(jobs);
    free(ids);
    return ok;
}

/* ---------------------------------------------------------------- flow head */

/* src/phonon_sampler.c:229-248 (mean_512): four interleaved 4-lane vectors,
 * two 16-group chunks, then the vectors and the lanes, in that order. */
float oracle_mean_512(const float input[512]) {
    float sums[4][4] = {{0}};
    for (size_t chunk = 0; chunk < 2; chunk++) {
        float partial[4][4] = {{0}};
        for (size_t group = 0; group < 16; group++)
            for (size_t v = 0; v < 4; v++)
                for (size_t lane = 0; lane < 4; lane++)
                    partial[v][lane] += input[chunk * 256 + group * 16 + v * 4 + lane];
        for (size_t v = 0; v < 4; v++)
            for (size_t lane = 0; lane < 4; lane++)
                sums[v][lane] += partial[v][lane];
    }
    for (size_t v = 1; v < 4; v++)
        for (size_t lane = 0; lane < 4; lane++)
            sums[0][lane] += sums[v][lane];
    float sum = 0.0f;
    for (size_t lane = 0; lane < 4; lane++)
        sum += sums[0][lane];
    return sum / 512.0f;
}

/* src/phonon_sampler.c:250-278: float mean (mean_512), variance from double
 * centred squares around it, eps 1e-6, optional affine. */
int oracle_flow_layer_norm(const float *input, const float *weight, const float *bias,
                           float output[512]) {
    if (!input || !output)
        return 0;
    for (size_t i = 0; i < 512; i++)
        if (!isfinite(input[i]) || (weight && !isfinite(weight[i])) ||
            (bias && !isfinite(bias[i])))
            return 0;
    const float mean = oracle_mean_512(input);
    double variance_sum = 0.0;
    for (size_t i = 0; i < 512; i++) {
        const double centred = (double)input[i] - mean;
        variance_sum += centred * centred;
    }
    const float variance = (float)(variance_sum / 512.0);
    const float inverse = 1.0f / sqrtf(variance + 1e-6f);
    for (size_t i = 0; i < 512; i++) {
        float v = (input[i] - mean) * inverse;
        if (weight)
            v = v * weight[i];
        if (bias)
            v = v + bias[i];
        output[i] = v;
        if (!isfinite(v))
            return 0;
    }
    return 1;
}

/* src/phonon_math.c:18-28: x / (1 + exp(-x)) (libm in place of SLEEF). */
int oracle_silu(float *values, size_t count) {
    if (!values)
        return 0;
    for (size_t i = 0; i < count; i++)
        values[i] = values[i] / (1.0f + expf(-values[i]));
    return 1;
}

/* src/phonon_sampler.c:280-305: [cos | sin](value * freqs) -> mlp.0 -> SiLU
 * -> mlp.2 -> alpha * out / sqrt(mean(out^2) + 1e-5) with mean_512. */
int oracle_time_embedding(const OracleFlowHead *head, size_t which, float value,
                          float output[512]) {
    if (!head || which > 1 || !output || !isfinite(value))
        return 0;
    float embedding[256], hidden[512], squares[512];
    for (size_t i = 0; i < 128; i++) {
        const float phase = value * head->time_freqs[which][i];
        embedding[i] = cosf(phase);
        embedding[128 + i] = sinf(phase);
    }
    if (!oracle_linear_batch(head->time_weight[which][0], embedding, 512, 256,
                             head->time_bias[which][0], hidden, 1) ||
        !oracle_silu(hidden, 512) ||
        !oracle_linear_batch(head->time_weight[which][1], hidden, 512, 512,
                             head->time_bias[which][1], output, 1))
        return 0;
    for (size_t i = 0; i < 512; i++)
        squares[i] = output[i] * output[i];
    const float inverse = 1.0f / sqrtf(oracle_mean_512(squares) + 1e-5f);
    for (size_t i = 0; i < 512; i++)
        output[i] = (head->time_alpha[which][i] * output[i]) * inverse;
    return 1;
}

/* h = LN(x) * (1 + scale) + shift, the adaLN modulation of
 * src/phonon_sampler.c:330-334 and :350-354. */
static void modulate(float h[512], const float *shift, const float *scale) {
    for (size_t i = 0; i < 512; i++) {
        const float one_plus_scale = 1.0f + scale[i];
        const float scaled = h[i] * one_plus_scale;
        h[i] = scaled + shift[i];
    }
}

/* src/phonon_sampler.c:307-359 (head_forward_cancel, without the cancel
 * poll). */
int oracle_flow_head_forward(const OracleFlowHead *head, const float condition[512],
                             const float state[32], float s, float t, float velocity[32]) {
    float x[512], y[512], time_s[512], time_t[512], modulation[1536];
    float h[512], first[512], second[512], normalized[512];
    if (!head || !condition || !state || !velocity || !isfinite(s) || !isfinite(t) ||
        !oracle_linear_batch(head->input_weight, state, 512, 32, head->input_bias, x, 1) ||
        !oracle_linear_batch(head->cond_weight, condition, 512, 512, head->cond_bias, y, 1) ||
        !oracle_time_embedding(head, 0, s, time_s) || !oracle_time_embedding(head, 1, t, time_t))
        return 0;
    for (size_t i = 0; i < 512; i++)
        y[i] += 0.5f * (time_s[i] + time_t[i]);
    for (size_t block = 0; block < ORACLE_HEAD_BLOCKS; block++) {
        memcpy(normalized, y, sizeof(normalized));
        oracle_silu(normalized, 512);
        if (!oracle_linear_batch(head->block_ada_weight[block], normalized, 1536, 512,
                                 head->block_ada_bias[block], modulation, 1) ||
            !oracle_flow_layer_norm(x, head->block_norm_weight[block],
                                    head->block_norm_bias[block], h))
            return 0;
        modulate(h, modulation, modulation + 512);
        if (!oracle_linear_batch(head->block_mlp_weight[block][0], h, 512, 512,
                                 head->block_mlp_bias[block][0], first, 1))
            return 0;
        oracle_silu(first, 512);
        if (!oracle_linear_batch(head->block_mlp_weight[block][1], first, 512, 512,
                                 head->block_mlp_bias[block][1], second, 1))
            return 0;
        for (size_t i = 0; i < 512; i++) {
            const float gated = modulation[1024 + i] * second[i];
            x[i] = x[i] + gated;
        }
    }
    memcpy(normalized, y, sizeof(normalized));
    oracle_silu(normalized, 512);
    if (!oracle_linear_batch(head->final_ada_weight, normalized, 1024, 512, head->final_ada_bias,
                             modulation, 1) ||
        !oracle_flow_layer_norm(x, NULL, NULL, h))
        return 0;
    modulate(h, modulation, modulation + 512);
    return oracle_linear_batch(head->final_weight, h, 32, 512, head->final_bias, velocity, 1);
}

/* src/phonon_sampler.c:366-393: one Euler step from temperature-scaled
 * noise at s = 0, t = 1. */
int oracle_lsd_one_step(const OracleFlowHead *head, const float condition[512],
                        const float raw_noise[32], float temperature, float output[32]) {
    float noise[32], velocity[32];
    if (!head || !condition || !raw_noise || !output || !isfinite(temperature) ||
        temperature <= 0.0f)
        return 0;
    const float scale = sqrtf(temperature);
    for (size_t i = 0; i < 32; i++) {
        if (!isfinite(raw_noise[i]))
            return 0;
        noise[i] = raw_noise[i] * scale;
    }
    if (!oracle_flow_head_forward(head, condition, noise, 0.0f, 1.0f, velocity))
        return 0;
    for (size_t i = 0; i < 32; i++) {
        output[i] = noise[i] + velocity[i];
        if (!isfinite(output[i]))
            return 0;
    }
    return 1;
}

/* src/phonon_sampler.c:395-401: the one-row affine flow_lm.out_eos. */
int oracle_eos_logit(const float *weight, const float *bias, const float state[512],
                     float *raw_logit) {
    return weight && bias && state && raw_logit &&
           oracle_linear_batch(weight, state, 1, 512, bias, raw_logit, 1);
}
