/* Device-resident Q8_0 matrices for repeated matvecs on the MI355X.
 *
 * No counterpart in the reference: phonon_q8_matvec (src/phonon_q8.c:64-92)
 * takes host blocks on every call. This interface uploads a matrix once (in
 * `copies` identical copies, so a benchmark can rotate through more bytes
 * than the 256 MB Infinity Cache holds) and runs the same arithmetic as
 * phonon_q8_matvec on device vectors. */
#ifndef PHONON_Q8_DEVICE_H
#define PHONON_Q8_DEVICE_H

#include "phonon_q8.h"
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct PhononQ8Device PhononQ8Device;

/* Upload `copies` copies of a [rows][columns] Q8_0 matrix (rows % 16 == 0,
 * columns % 32 == 0). Fails on a non-finite scale. */
int phonon_q8_device_create(const PhononQ8Block *weights, size_t rows, size_t columns,
                            size_t copies, PhononQ8Device **matrix);
void phonon_q8_device_destroy(PhononQ8Device *matrix);
/* y[b][r] = dot(row r of copy `copy`, x[b]) for b < batch, with x (dev)
 * [batch][columns] and y (dev) [batch][rows], both 16-byte aligned,
 * enqueued on `stream` (a HIP stream, NULL = null stream). With 512 columns
 * the projection splits the fp32 rows itself (one launch); otherwise the
 * input is first converted to split fragments in a buffer owned by the
 * matrix, so calls on one matrix must not overlap in time. Returns 0 on
 * invalid arguments (a misaligned pointer included) or a failed launch;
 * non-finite outputs are reported by phonon_q8_device_status. */
int phonon_q8_device_matvec(PhononQ8Device *matrix, size_t copy, const float *x, float *y,
                            size_t batch, void *stream);
/* The same product for batch <= 8 on the vector units (pgpu_q8_gemv: one
 * lane per 32-column block of a row, 16-byte int8 loads from a row-major
 * copy made at creation, the reference's arithmetic, so y has the bits of
 * phonon_q8_matvec). Columns must be 32 x a divisor of 64; returns 0
 * otherwise. */
int phonon_q8_device_matvec_valu(PhononQ8Device *matrix, size_t copy, const float *x, float *y,
                                 size_t batch, void *stream);
/* Waits for `stream`; 1 iff no call since the last check produced a
 * non-finite output (and clears the record). */
int phonon_q8_device_status(PhononQ8Device *matrix, void *stream);
/* Algorithmic bytes of one matvec call: weights + input + output. */
size_t phonon_q8_device_bytes_per_call(const PhononQ8Device *matrix, size_t batch);

#ifdef __cplusplus
}
#endif

#endif
