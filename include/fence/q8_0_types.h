/*
 * fence/q8_0_types.h -- the Q8_0 block as the reference declares it
 * (src/kernels/q8_0_types.h:8-17): an fp16 scale followed by 32 int8 values,
 * 34 bytes with no padding.  The layout is the GGUF on-disk format, so it must
 * match byte for byte.
 */
#ifndef FENCE_Q8_0_TYPES_H
#define FENCE_Q8_0_TYPES_H

#include <stdint.h>
#include <hip/hip_fp16.h>

#define QK8_0 32

#pragma pack(push, 1)
struct block_q8_0 {
    __half d;           /* scale */
    int8_t qs[QK8_0];   /* quants */
};
#pragma pack(pop)

static_assert(sizeof(block_q8_0) == 34, "block_q8_0 must be 34 bytes");

#endif /* FENCE_Q8_0_TYPES_H */
