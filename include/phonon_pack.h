/* Tensor-view types of speech-mac src/phonon_pack.h:9-19, which the
 * transformer boundary takes as weights. Only the types cross this
 * boundary: the kpack file loader itself is not part of this library. */
#ifndef PHONON_PACK_H
#define PHONON_PACK_H

#include <stddef.h>
#include <stdint.h>

#define PHONON_PACK_MAX_RANK 8

/* Replaces PhononPackDType, src/phonon_pack.h:9. */
typedef enum { PHONON_PACK_Q8_0 = 1, PHONON_PACK_BF16 = 2 } PhononPackDType;

/* Replaces PhononTensorView, src/phonon_pack.h:10-19. `linear_data` (an fp32
 * materialization) is accepted and ignored: the device path consumes the
 * packed Q8_0/BF16 bytes directly. */
typedef struct {
    PhononPackDType dtype;
    unsigned int rank;
    uint64_t shape[PHONON_PACK_MAX_RANK];
    const void *data;
    size_t byte_count;
    const float *linear_data;
} PhononTensorView;

#endif
