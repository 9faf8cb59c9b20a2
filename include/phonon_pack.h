/* Drop-in replacement for speech-mac src/phonon_pack.h (src/phonon_pack.h:
 * 1-38): the kpack v1 loader and its tensor views, which the transformer
 * boundary takes as weights. The views point into the pack's file image;
 * phonon_flow_model_create / phonon_flow_prepare_weights upload them to the
 * MI355X (Q8_0 repacked into MFMA fragment order). Same signatures and
 * 1 = success / 0 = failure convention as the reference. */
#ifndef PHONON_PACK_H
#define PHONON_PACK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PHONON_PACK_MAX_RANK 8

/* Replaces PhononPackDType, src/phonon_pack.h:9. */
typedef enum { PHONON_PACK_Q8_0 = 1, PHONON_PACK_BF16 = 2 } PhononPackDType;

/* Replaces PhononTensorView, src/phonon_pack.h:10-19. `linear_data` (an fp32
 * materialization, phonon_pack_prepare_linears) is kept for the reference's
 * callers; the device path consumes the packed Q8_0/BF16 bytes directly. */
typedef struct {
    PhononPackDType dtype;
    unsigned int rank;
    uint64_t shape[PHONON_PACK_MAX_RANK];
    const void *data;
    size_t byte_count;
    const float *linear_data;
} PhononTensorView;

/* Replaces PhononPack, src/phonon_pack.h:20. */
typedef struct PhononPack PhononPack;

/* src/phonon_pack.h:22-23 (src/phonon_pack.c:87-290): reads and validates a
 * kpack v1 file (header, the pinned model and config digests, SHA-256 of
 * index, metadata and payload, the pinned index digest, 36 Q8_0 + 173 BF16
 * tensors with unique names and non-overlapping aligned ranges). Names and
 * data are borrowed from the pack until phonon_pack_close. */
int phonon_pack_open(const char *path, PhononPack **pack);
void phonon_pack_close(PhononPack *pack);
/* src/phonon_pack.h:24-28 (src/phonon_pack.c:413-448): fp32 materialization
 * of every rank-2 linear (not lookup tables or the unused flow.w_s_t
 * branch), at most 256 MiB; idempotent; a failure keeps none. */
int phonon_pack_prepare_linears(PhononPack *pack);
/* src/phonon_pack.h:29-31 (src/phonon_pack.c:372-411). */
int phonon_tensor_expand_linear(const PhononTensorView *view, float **output);
/* src/phonon_pack.h:32-35. */
size_t phonon_pack_tensor_count(const PhononPack *pack);
int phonon_pack_tensor(const PhononPack *pack, const char *name, PhononTensorView *view);
int phonon_pack_tensor_at(const PhononPack *pack, size_t index, const char **name,
                          size_t *name_length, PhononTensorView *view);
/* src/phonon_pack.h:36-37 (src/phonon_pack.c:321-341): fails on overlap or a
 * non-finite value. */
int phonon_bf16_to_float(const uint16_t *values, size_t count, float *output);

/* Test seams of tests/phonon_pack_test.h:7-10 (src/phonon_pack.c:292,450):
 * open without pinning the published model's index digest (synthetic
 * packs), and prepare_linears with a byte limit. */
int phonon_pack_open_for_tests(const char *path, PhononPack **pack);
int phonon_pack_prepare_linears_for_tests(PhononPack *pack, size_t limit);

#ifdef __cplusplus
}
#endif

#endif
