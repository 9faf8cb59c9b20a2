/* Library-wide state of libphonon_mi355x: device selection, the HIP stream
 * and scratch of the single-stream API, weight repacking and RoPE tables. */
#include "ph_internal.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static pthread_once_t g_once = PTHREAD_ONCE_INIT;
static int g_ready;
static void *g_stream;

static void init_once(void) {
    if (!pgpu_device_init())
        return;
    if (!pgpu_stream_create(&g_stream))
        return;
    g_ready = 1;
}

int ph_init(void) {
    pthread_once(&g_once, init_once);
    return g_ready;
}

void *ph_stream(void) { return g_stream; }

int ph_fail(const char *why) {
    char text[256];
    const char *prior = pgpu_last_error();
    snprintf(text, sizeof(text), "%s%s%s", why, prior && *prior ? " <- " : "",
             prior ? prior : "");
    pgpu_record_error(text);
    return 0;
}
void ph_lock(void) { pthread_mutex_lock(&g_lock); }
void ph_unlock(void) { pthread_mutex_unlock(&g_lock); }

static void *g_scratch[8];
static size_t g_scratch_bytes[8];

void *ph_scratch(int slot, size_t bytes) {
    if (slot < 0 || slot >= 8)
        return NULL;
    if (g_scratch_bytes[slot] < bytes) {
        if (g_scratch[slot] && !pgpu_stream_sync(g_stream))
            return NULL;
        pgpu_free(g_scratch[slot]);
        g_scratch[slot] = pgpu_malloc(bytes);
        g_scratch_bytes[slot] = g_scratch[slot] ? bytes : 0;
    }
    return g_scratch[slot];
}

static float from_bits(uint32_t bits) {
    float f;
    memcpy(&f, &bits, sizeof(f));
    return f;
}

float ph_half_to_float(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits >> 15) << 31;
    uint32_t exponent = (bits >> 10) & 31u, fraction = bits & 1023u;
    if (exponent == 31u)
        return from_bits(sign | 0x7f800000u | (fraction << 13));
    if (exponent)
        return from_bits(sign | ((exponent + 112u) << 23) | (fraction << 13));
    if (!fraction)
        return from_bits(sign);
    exponent = 113u;
    while (!(fraction & 1024u)) {
        fraction <<= 1;
        exponent--;
    }
    return from_bits(sign | (exponent << 23) | ((fraction & 1023u) << 13));
}

int ph_half_finite(uint16_t bits) { return ((bits >> 10) & 31u) != 31u; }
int ph_bf16_finite(uint16_t bits) { return ((bits >> 7) & 0xffu) != 0xffu; }
float ph_bf16_to_float(uint16_t bits) { return from_bits((uint32_t)bits << 16); }

int ph_all_finite(const float *values, size_t count) {
    for (size_t i = 0; i < count; i++)
        if (!isfinite(values[i]))
            return 0;
    return 1;
}

int ph_overlap(const void *a, size_t a_bytes, const void *b, size_t b_bytes) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + b_bytes && y < x + a_bytes;
}

/* Q8_0 block of the reference layout (src/phonon_q8.h:12-17). */
static const PhononQ8Block *q8_block(const PhononTensorView *view, size_t row, size_t kb,
                                     size_t per_row) {
    return (const PhononQ8Block *)view->data + row * per_row + kb;
}

int ph_matrix_upload(const PhononTensorView *view, size_t rows, size_t columns,
                     pgpu_matrix *out, void **device) {
    *device = NULL;
    if (!view || !view->data || view->rank != 2 || view->shape[0] != rows ||
        view->shape[1] != columns || !rows || !columns)
        return 0;
    const int q8 = view->dtype == PHONON_PACK_Q8_0;
    if (q8) {
        if (columns % 32 || view->byte_count != rows * columns / 32 * sizeof(PhononQ8Block))
            return 0;
    } else if (view->dtype != PHONON_PACK_BF16 ||
               view->byte_count != rows * columns * sizeof(uint16_t)) {
        return 0;
    }
    const size_t prow = (rows + 15) / 16 * 16, pcol = (columns + 31) / 32 * 32;
    const size_t tiles = prow / 16, kbn = pcol / 32;
    const size_t value_bytes = prow * pcol * (q8 ? 1 : 2);
    const size_t scale_bytes = q8 ? prow * kbn * sizeof(uint16_t) : 0;
    unsigned char *host = calloc(1, value_bytes + scale_bytes);
    if (!host)
        return 0;
    int ok = 1;
    if (q8) {
        int8_t *values = (int8_t *)host;
        uint16_t *scales = (uint16_t *)(host + value_bytes);
        for (size_t t = 0; t < tiles && ok; t++)
            for (size_t kb = 0; kb < kbn && ok; kb++) {
                int8_t *record = values + (t * kbn + kb) * 512;
                for (size_t r = 0; r < 16; r++) {
                    const size_t row = t * 16 + r;
                    if (row >= rows)
                        continue;
                    const PhononQ8Block *b = q8_block(view, row, kb, columns / 32);
                    if (!ph_half_finite(b->scale_bits)) {
                        ok = 0;
                        break;
                    }
                    scales[(t * kbn + kb) * 16 + r] = b->scale_bits;
                    for (size_t g = 0; g < 4; g++)
                        memcpy(record + (g * 16 + r) * 8, b->values + g * 8, 8);
                }
            }
    } else {
        const uint16_t *src = view->data;
        uint16_t *values = (uint16_t *)host;
        for (size_t t = 0; t < tiles && ok; t++)
            for (size_t kb = 0; kb < kbn && ok; kb++) {
                uint16_t *record = values + (t * kbn + kb) * 512;
                for (size_t r = 0; r < 16; r++) {
                    const size_t row = t * 16 + r;
                    if (row >= rows)
                        continue;
                    for (size_t c = 0; c < 32; c++) {
                        const size_t col = kb * 32 + c;
                        if (col >= columns)
                            continue;
                        const uint16_t w = src[row * columns + col];
                        if (!ph_bf16_finite(w))
                            ok = 0;
                        record[((c / 8) * 16 + r) * 8 + c % 8] = w;
                    }
                }
            }
    }
    void *dev = ok ? pgpu_malloc(value_bytes + scale_bytes) : NULL;
    if (dev && !pgpu_copy_h2d(ph_stream(), dev, host, value_bytes + scale_bytes)) {
        pgpu_free(dev);
        dev = NULL;
    }
    free(host);
    if (!dev)
        return 0;
    out->q8 = q8;
    out->rows = prow;
    out->columns = pcol;
    out->values = dev;
    out->scales = q8 ? (const uint16_t *)((unsigned char *)dev + value_bytes) : NULL;
    *device = dev;
    return 1;
}

int ph_vector_decode(const PhononTensorView *view, size_t count, float *host) {
    if (!view || !view->data || view->rank != 1 || view->shape[0] != count ||
        view->dtype != PHONON_PACK_BF16 || view->byte_count != count * sizeof(uint16_t))
        return 0;
    const uint16_t *bits = view->data;
    for (size_t i = 0; i < count; i++) {
        if (!ph_bf16_finite(bits[i]))
            return 0;
        host[i] = ph_bf16_to_float(bits[i]);
    }
    return 1;
}

void ph_rope_row(float theta, size_t position, size_t head_width, float *cos_sin) {
    for (size_t i = 0; i < head_width / 2; i++) {
        const float exponent = (float)(2 * i) / (float)head_width;
        const float freq = 1.0f / powf(theta, exponent);
        const float phase = (float)position * freq;
        cos_sin[2 * i] = cosf(phase);
        cos_sin[2 * i + 1] = sinf(phase);
    }
}

/* Tables are immutable once built (captured graphs keep their address), one
 * per (theta, length), kept until the process ends. */
enum { ROPE_TABLES = 8 };
static pthread_mutex_t g_rope_lock = PTHREAD_MUTEX_INITIALIZER;
static float g_rope_theta[ROPE_TABLES];
static size_t g_rope_rows[ROPE_TABLES];
static float *g_rope_dev[ROPE_TABLES];

static const float *rope_table(float theta, size_t rows) {
    if (!(theta > 0.0f) || !isfinite(theta))
        return NULL;
    pthread_mutex_lock(&g_rope_lock);
    const float *found = NULL;
    size_t slot = 0;
    for (; slot < ROPE_TABLES && g_rope_dev[slot]; slot++)
        if (g_rope_theta[slot] == theta && g_rope_rows[slot] == rows) {
            found = g_rope_dev[slot];
            break;
        }
    if (!found && slot < ROPE_TABLES) {
        const size_t floats = rows * 32 * 2;
        float *host = malloc(floats * sizeof(float));
        float *dev = host ? pgpu_malloc(floats * sizeof(float)) : NULL;
        if (dev) {
            for (size_t p = 0; p < rows; p++)
                ph_rope_row(theta, p, 64, host + p * 64);
            if (pgpu_copy_h2d(g_stream, dev, host, floats * sizeof(float)) &&
                pgpu_stream_sync(g_stream)) {
                g_rope_theta[slot] = theta;
                g_rope_rows[slot] = rows;
                g_rope_dev[slot] = dev;
                found = dev;
            } else {
                pgpu_free(dev);
            }
        }
        free(host);
    }
    pthread_mutex_unlock(&g_rope_lock);
    return found;
}

const float *ph_rope_table(float theta) { return rope_table(theta, PHONON_FLOW_MAX_POSITIONS); }

const float *ph_rope_table_long(float theta) { return rope_table(theta, PH_ROPE_LONG_ROWS); }
