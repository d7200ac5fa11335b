/*
 * quant.h -- ggml quantised block formats used by the model and their scalar
 * dequantisation.  Drop-in for the reference include/quant.h:1-87.
 * The block layouts are the ggml on-disk format and are reproduced field for
 * field (sizes asserted below); host/quant.c is this library's own code.
 */
#if !defined(QWEN_QUANT_H) && !defined(QUANT_H)   /* either header, whichever came first */
#define QWEN_QUANT_H
/* the reference header of the same name is superseded by this one when both
   are on the include path (reference drivers compiled against this library) */
#define QUANT_H

#include "gguf.h"
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QK_K  256          /* elements per K-quant / IQ4_XS super-block */
#define QK8_0 32           /* elements per Q8_0 block */

typedef uint16_t fp16_t;
float fp16_to_f32(fp16_t h);   /* exact, subnormals included (reference quant.c:6-28) */

typedef struct { fp16_t d; int8_t qs[QK8_0]; } block_q8_0;                     /* 34 B  */
typedef struct { fp16_t d, dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; } block_q4_K;   /* 144 B */
typedef struct { fp16_t d, dmin; uint8_t scales[12]; uint8_t qh[QK_K / 8];
                 uint8_t qs[QK_K / 2]; } block_q5_K;                              /* 176 B */
typedef struct { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16];
                 fp16_t d; } block_q6_K;                                          /* 210 B */
typedef struct { fp16_t d; uint16_t scales_h; uint8_t scales_l[QK_K / 64];
                 uint8_t qs[QK_K / 2]; } block_iq4_xs;                            /* 136 B */

#ifndef __cplusplus
_Static_assert(sizeof(block_q8_0) == 34, "q8_0");
_Static_assert(sizeof(block_q4_K) == 144, "q4_K");
_Static_assert(sizeof(block_q5_K) == 176, "q5_K");
_Static_assert(sizeof(block_q6_K) == 210, "q6_K");
_Static_assert(sizeof(block_iq4_xs) == 136, "iq4_xs");
#endif

/* 6-bit (scale, min) pair j of a Q4_K/Q5_K block (reference quant.h:21-29) */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m)
{
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

extern const int8_t kvalues_iq4nl[16];     /* IQ4_NL codebook (reference quant.c:30-32) */

size_t quant_block_size(ggml_type_t t);                       /* quant.c:34-45 */
size_t quant_row_bytes(ggml_type_t t, uint64_t ne0);          /* quant.c:61-65 */
const void *quant_row_ptr(const gguf_tensor_info_t *t, uint64_t row);   /* quant.c:67-69 */
/* scalar reference dequantisation of one row; 0 ok, -1 unsupported (quant.c:184-208) */
int dequant_row(ggml_type_t t, const void *data, uint64_t ne0, float *dst);
const char *quant_type_name(ggml_type_t t);                   /* quant.c:71-82 */

#ifdef __cplusplus
}
#endif
#endif
