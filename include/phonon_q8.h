/* Drop-in replacement for speech-mac src/phonon_q8.h (src/phonon_q8.h:1-21).
 * Same block type, same signatures, same 1/0 return convention; the
 * implementation (libphonon_mi355x) runs the matvec on the MI355X. */
#ifndef PHONON_Q8_H
#define PHONON_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML Q8_0 block: little-endian IEEE binary16 scale, then 32 signed values.
 * Replaces PhononQ8Block, src/phonon_q8.h:12-17 (34 bytes, packed). */
typedef struct {
    uint16_t scale_bits;
    int8_t values[32];
} PhononQ8Block;

#ifdef __cplusplus
static_assert(sizeof(PhononQ8Block) == 34, "Q8_0 blocks are 34 bytes");
#else
_Static_assert(sizeof(PhononQ8Block) == 34, "Q8_0 blocks are 34 bytes");
#endif

/* Replaces phonon_q8_dot, src/phonon_q8.c:36-62: result = sum over blocks of
 * scale * (sum of q*x). Fails (returns 0) on NULL, elements%32, a
 * non-finite scale, input or result. */
int phonon_q8_dot(const PhononQ8Block *blocks, const float *input, size_t elements,
                  float *result);

/* Replaces phonon_q8_matvec, src/phonon_q8.c:64-92: output[r] = dot(row r, input).
 * Buffers are host memory and borrowed. Input/output and weights/output must
 * not overlap. Output contents are unspecified on failure. */
int phonon_q8_matvec(const PhononQ8Block *weights, const float *input, size_t rows,
                     size_t columns, float *output);

#ifdef __cplusplus
}
#endif

#endif
