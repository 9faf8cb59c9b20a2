/* phonon_q8_dot / phonon_q8_matvec on the MI355X (phonon_q8.h), and the
 * device-resident matrices of phonon_q8_device.h.
 *
 * Argument checks follow src/phonon_q8.c:36-92. The arithmetic per row is
 * the reference's: for every 32-column block, partial = sum q*x, then
 * sum += scale * partial. The drop-ins and phonon_q8_device_matvec_valu
 * run it on the vector units with the reference's rounding order
 * (pgpu_gemv.hip: the same bits); phonon_q8_device_matvec runs it on the
 * matrix cores (each block's partial from exact split bf16 MFMA terms,
 * pgpu_gemm.hip), and the drop-in matvec falls back to that path when the
 * column count is not 32 x a divisor of 64. */
#include "phonon_q8_device.h"
#include "ph_internal.h"

#include <stdlib.h>
#include <string.h>

struct PhononQ8Device {
    pgpu_matrix *copies;
    void **allocations;
    int8_t **row_values;   /* per copy: row-major int8 [rows][columns] */
    uint16_t **row_scales; /* per copy: fp16 bits [rows][columns/32] */
    size_t count, rows, columns, max_batch;
    uint16_t *xs;
    int *status;
};

void phonon_q8_device_destroy(PhononQ8Device *m) {
    if (!m)
        return;
    (void)pgpu_stream_sync(NULL);
    for (size_t i = 0; i < m->count; i++) {
        pgpu_free(m->allocations[i]);
        if (m->row_values)
            pgpu_free(m->row_values[i]);
        if (m->row_scales)
            pgpu_free(m->row_scales[i]);
    }
    free(m->row_values);
    free(m->row_scales);
    pgpu_free(m->xs);
    pgpu_free(m->status);
    free(m->copies);
    free(m->allocations);
    free(m);
}

int phonon_q8_device_create(const PhononQ8Block *weights, size_t rows, size_t columns,
                            size_t copies, PhononQ8Device **matrix) {
    if (!matrix)
        return 0;
    *matrix = NULL;
    if (!weights || !rows || rows % 16 || !columns || columns % 32 || !copies ||
        copies > 100000 || rows > SIZE_MAX / columns || !ph_init())
        return 0;
    PhononQ8Device *m = calloc(1, sizeof(*m));
    if (!m)
        return 0;
    m->copies = calloc(copies, sizeof(pgpu_matrix));
    m->allocations = calloc(copies, sizeof(void *));
    m->rows = rows;
    m->columns = columns;
    m->max_batch = 64;
    PhononTensorView view = {.dtype = PHONON_PACK_Q8_0,
                             .rank = 2,
                             .shape = {rows, columns},
                             .data = weights,
                             .byte_count = rows * columns / 32 * sizeof(PhononQ8Block)};
    m->row_values = calloc(copies, sizeof(int8_t *));
    m->row_scales = calloc(copies, sizeof(uint16_t *));
    const size_t nb = columns / 32;
    int8_t *rv = malloc(rows * columns);
    uint16_t *rs = malloc(rows * nb * sizeof(uint16_t));
    int ok = m->copies && m->allocations && m->row_values && m->row_scales && rv && rs;
    for (size_t i = 0; ok && i < rows * nb; i++) {
        memcpy(rv + i * 32, weights[i].values, 32);
        rs[i] = weights[i].scale_bits;
    }
    for (size_t i = 0; ok && i < copies; i++) {
        ok = ph_matrix_upload(&view, rows, columns, &m->copies[i], &m->allocations[i]);
        if (ok)
            m->count++;
        ok = ok && (m->row_values[i] = pgpu_malloc(rows * columns)) &&
             (m->row_scales[i] = pgpu_malloc(rows * nb * sizeof(uint16_t))) &&
             pgpu_copy_h2d(NULL, m->row_values[i], rv, rows * columns) &&
             pgpu_copy_h2d(NULL, m->row_scales[i], rs, rows * nb * sizeof(uint16_t));
    }
    free(rv);
    free(rs);
    const size_t split_bytes = m->max_batch * (ok ? m->copies[0].columns : 0) * 3 * 2;
    if (ok) {
        m->xs = pgpu_malloc(split_bytes);
        m->status = pgpu_malloc(sizeof(int));
        ok = m->xs && m->status && pgpu_memset(NULL, m->xs, 0, split_bytes) &&
             pgpu_memset(NULL, m->status, 0, sizeof(int)) && pgpu_stream_sync(NULL);
    }
    if (!ok) {
        phonon_q8_device_destroy(m);
        return 0;
    }
    *matrix = m;
    return 1;
}

int phonon_q8_device_matvec(PhononQ8Device *m, size_t copy, const float *x, float *y,
                            size_t batch, void *stream) {
    /* The kernels read x and write y 16 bytes at a time. */
    if (!m || copy >= m->count || !x || !y || !batch || batch > m->max_batch ||
        (uintptr_t)x % 16 || (uintptr_t)y % 16)
        return 0;
    const pgpu_matrix *w = &m->copies[copy];
    if (w->columns != m->columns)
        return 0; /* padded columns would need a padded input */
    /* 512 columns: one launch that splits the rows inside the projection. */
    if (w->columns == PH_WIDTH) {
        const pgpu_gemm_input rows = {.rows = x};
        return pgpu_gemm_store(stream, w, &rows, (int)batch, NULL, y, (int)w->rows, m->status);
    }
    const pgpu_gemm_input in = {.split = m->xs};
    return pgpu_split_rows(stream, x, (int)batch, (int)w->columns, m->xs, m->status) &&
           pgpu_gemm_store(stream, w, &in, (int)batch, NULL, y, (int)w->rows, m->status);
}

int phonon_q8_device_matvec_valu(PhononQ8Device *m, size_t copy, const float *x, float *y,
                                 size_t batch, void *stream) {
    if (!m || copy >= m->count || !x || !y || !batch || batch > PGPU_GEMV_MAX_BATCH ||
        (uintptr_t)x % 16 || (uintptr_t)y % 16)
        return 0;
    return pgpu_q8_gemv(stream, m->row_values[copy], m->row_scales[copy], (int)m->rows,
                        (int)m->columns, x, (int)batch, y, m->status);
}

int phonon_q8_device_status(PhononQ8Device *m, void *stream) {
    int st = 1;
    if (!m || !pgpu_stream_sync(stream) || !pgpu_copy_d2h(stream, &st, m->status, sizeof(int)))
        return 0;
    if (st && !(pgpu_memset(stream, m->status, 0, sizeof(int)) && pgpu_stream_sync(stream)))
        return 0;
    return st == 0;
}

size_t phonon_q8_device_bytes_per_call(const PhononQ8Device *m, size_t batch) {
    if (!m)
        return 0;
    return m->rows * m->columns / 32 * sizeof(PhononQ8Block) +
           batch * (m->columns + m->rows) * sizeof(float);
}

/* ------------------------------------------------------------- drop-ins -- */

/* The reference's matvec on the vector units (pgpu_q8_gemv): the row-major
 * int8 values and fp16 scales of the blocks go to the device, and every
 * output has the bits of src/phonon_q8.c:64-92. Arguments already checked. */
static int q8_matvec_valu(const PhononQ8Block *weights, const float *input, size_t rows,
                          size_t columns, float *output) {
    const size_t nb = columns / 32, blocks = rows * nb;
    int8_t *rv = malloc(rows * columns);
    uint16_t *rs = malloc(blocks * sizeof(uint16_t));
    int ok = rv && rs;
    for (size_t i = 0; ok && i < blocks; i++) {
        memcpy(rv + i * 32, weights[i].values, 32);
        rs[i] = weights[i].scale_bits;
    }
    ph_lock();
    void *s = ph_stream();
    int8_t *dv = ok ? ph_scratch(4, rows * columns) : NULL;
    uint16_t *ds = ok ? ph_scratch(5, blocks * sizeof(uint16_t)) : NULL;
    float *x = ok ? ph_scratch(2, columns * sizeof(float)) : NULL;
    float *y = ok ? ph_scratch(3, rows * sizeof(float)) : NULL;
    int *status = ph_scratch(1, sizeof(int));
    int st = 1;
    ok = ok && dv && ds && x && y && status && pgpu_memset(s, status, 0, sizeof(int)) &&
         pgpu_copy_h2d(s, dv, rv, rows * columns) &&
         pgpu_copy_h2d(s, ds, rs, blocks * sizeof(uint16_t)) &&
         pgpu_copy_h2d(s, x, input, columns * sizeof(float)) &&
         pgpu_q8_gemv(s, dv, ds, (int)rows, (int)columns, x, 1, y, status) &&
         pgpu_copy_d2h(s, &st, status, sizeof(int)) &&
         pgpu_copy_d2h(s, output, y, rows * sizeof(float));
    (void)pgpu_stream_sync(s);
    ph_unlock();
    free(rv);
    free(rs);
    return ok && st == 0;
}

int phonon_q8_matvec(const PhononQ8Block *weights, const float *input, size_t rows,
                     size_t columns, float *output) {
    if (weights == NULL || input == NULL || output == NULL || rows == 0 || columns == 0 ||
        columns % 32 != 0 || rows > SIZE_MAX / (columns / 32) ||
        columns > SIZE_MAX / sizeof(*input) || rows > SIZE_MAX / sizeof(*output))
        return 0;
    const size_t input_bytes = columns * sizeof(float), output_bytes = rows * sizeof(float);
    const size_t blocks = rows * (columns / 32);
    if (blocks > SIZE_MAX / sizeof(PhononQ8Block))
        return 0;
    const size_t weight_bytes = blocks * sizeof(PhononQ8Block);
    if ((uintptr_t)input > UINTPTR_MAX - input_bytes ||
        (uintptr_t)output > UINTPTR_MAX - output_bytes ||
        (uintptr_t)weights > UINTPTR_MAX - weight_bytes ||
        ph_overlap(input, input_bytes, output, output_bytes) ||
        ph_overlap(weights, weight_bytes, output, output_bytes))
        return 0;
    /* The reference fails on the first non-finite scale or input. */
    if (!ph_all_finite(input, columns))
        return 0;
    for (size_t i = 0; i < blocks; i++)
        if (!ph_half_finite(weights[i].scale_bits))
            return 0;
    if (rows > INT32_MAX / 2 || columns > INT32_MAX / 2 || !ph_init())
        return 0;
    const size_t nb = columns / 32;
    if (nb <= 64 && 64 % nb == 0)
        return q8_matvec_valu(weights, input, rows, columns, output);
    ph_lock();
    void *s = ph_stream();
    pgpu_matrix w;
    void *wdev = NULL;
    PhononTensorView view = {.dtype = PHONON_PACK_Q8_0,
                             .rank = 2,
                             .shape = {rows, columns},
                             .data = weights,
                             .byte_count = weight_bytes};
    int ok = ph_matrix_upload(&view, rows, columns, &w, &wdev);
    float *x = ok ? ph_scratch(2, columns * sizeof(float)) : NULL;
    float *y = ok ? ph_scratch(3, w.rows * sizeof(float)) : NULL;
    uint16_t *xs = ok ? ph_scratch(5, 16 * columns * 3 * sizeof(uint16_t)) : NULL;
    int *status = ph_scratch(1, sizeof(int));
    float *host = ok ? malloc(w.rows * sizeof(float)) : NULL;
    int st = 1;
    const pgpu_gemm_input in = {.split = xs};
    ok = ok && x && y && xs && status && host && pgpu_memset(s, status, 0, sizeof(int)) &&
         pgpu_memset(s, xs, 0, 16 * columns * 3 * sizeof(uint16_t)) &&
         pgpu_copy_h2d(s, x, input, input_bytes) &&
         pgpu_split_rows(s, x, 1, (int)columns, xs, status) &&
         pgpu_gemm_store(s, &w, &in, 1, NULL, y, (int)w.rows, status) &&
         pgpu_copy_d2h(s, &st, status, sizeof(int)) &&
         pgpu_copy_d2h(s, host, y, w.rows * sizeof(float));
    if (ok && st == 0)
        memcpy(output, host, output_bytes);
    (void)pgpu_stream_sync(s);
    pgpu_free(wdev);
    ph_unlock();
    free(host);
    return ok && st == 0;
}

int phonon_q8_dot(const PhononQ8Block *blocks, const float *input, size_t elements,
                  float *result) {
    if (blocks == NULL || input == NULL || result == NULL || elements == 0 ||
        elements % 32 != 0 || elements / 32 > SIZE_MAX / sizeof(*blocks) ||
        elements > SIZE_MAX / sizeof(*input))
        return 0;
    const size_t block_bytes = elements / 32 * sizeof(*blocks);
    const size_t input_bytes = elements * sizeof(*input);
    if ((uintptr_t)blocks > UINTPTR_MAX - block_bytes ||
        (uintptr_t)input > UINTPTR_MAX - input_bytes)
        return 0;
    float out;
    if (!phonon_q8_matvec(blocks, input, 1, elements, &out))
        return 0;
    *result = out;
    return 1;
}
