/*
 * fence/q6k_types.h -- the Q6_K super-block as the reference declares it
 * (src/kernels/q6k_types.h:21-39): 256 weights in 210 bytes -- the low
 * nibbles ql[128], the high two bits qh[64], 16 int8 sub-block scales and an
 * fp16 super-block scale, packed.  The layout is the GGUF on-disk format, so
 * it must match byte for byte.
 */
#ifndef FENCE_Q6K_TYPES_H
#define FENCE_Q6K_TYPES_H

#include <stdint.h>
#include <hip/hip_fp16.h>

#define QK_K 256

#pragma pack(push, 1)
struct block_q6_K {
    uint8_t ql[QK_K / 2];      /* low four bits of each quant */
    uint8_t qh[QK_K / 4];      /* high two bits of each quant */
    int8_t scales[QK_K / 16];  /* sub-block scales */
    __half d;                  /* super-block scale */
};
#pragma pack(pop)

static_assert(sizeof(block_q6_K) == 210, "block_q6_K must be 210 bytes");

#endif /* FENCE_Q6K_TYPES_H */
