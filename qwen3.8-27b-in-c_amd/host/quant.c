/*
 * quant.c -- host-side block-format helpers and scalar dequantisation
 * (the reference API of include/quant.h).  The GPU path decodes the same
 * blocks in csrc/ (bit-identical: every weight is one correctly rounded
 * product, see dequant_row below); this file serves host callers such as the
 * embedding fetch of the drop-in API and the weight packer.
 */
#include "quant.h"
#include <string.h>

const int8_t kvalues_iq4nl[16] = { -127, -104, -83, -65, -49, -35, -22, -10,
                                   1, 13, 25, 38, 53, 69, 89, 113 };

float fp16_to_f32(fp16_t h)
{
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
    if (e == 0x1F) {
        u = s | 0x7F800000u | (m << 13);
    } else if (e) {
        u = s | ((e + 112u) << 23) | (m << 13);
    } else if (!m) {
        u = s;
    } else {                                   /* subnormal half -> normal float */
        int sh = __builtin_clz(m) - 21;        /* bring bit 10 to the top */
        m = (m << sh) & 0x3FFu;
        u = s | ((uint32_t)(113 - sh) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

size_t quant_block_size(ggml_type_t t)
{
    switch (t) {
    case GGML_F32: return 4;
    case GGML_F16: return 2;
    case GGML_Q8_0: return sizeof(block_q8_0);
    case GGML_Q4_K: return sizeof(block_q4_K);
    case GGML_Q5_K: return sizeof(block_q5_K);
    case GGML_Q6_K: return sizeof(block_q6_K);
    case GGML_IQ4_XS: return sizeof(block_iq4_xs);
    default: return 0;
    }
}

static uint64_t block_elems(ggml_type_t t)
{
    switch (t) {
    case GGML_F32: case GGML_F16: return 1;
    case GGML_Q8_0: return QK8_0;
    case GGML_Q4_K: case GGML_Q5_K: case GGML_Q6_K: case GGML_IQ4_XS: return QK_K;
    default: return 0;
    }
}

size_t quant_row_bytes(ggml_type_t t, uint64_t ne0)
{
    const uint64_t be = block_elems(t);
    return be ? (size_t)(ne0 / be) * quant_block_size(t) : 0;
}

const void *quant_row_ptr(const gguf_tensor_info_t *t, uint64_t row)
{
    return (const uint8_t *)t->data + (size_t)row * quant_row_bytes(t->type, t->ne[0]);
}

const char *quant_type_name(ggml_type_t t)
{
    switch (t) {
    case GGML_F32: return "F32";
    case GGML_F16: return "F16";
    case GGML_Q8_0: return "Q8_0";
    case GGML_Q4_K: return "Q4_K";
    case GGML_Q5_K: return "Q5_K";
    case GGML_Q6_K: return "Q6_K";
    case GGML_IQ4_XS: return "IQ4_XS";
    default: return "UNSUPPORTED";
    }
}

/* Each element is produced with the same roundings as the reference scalar
 * decoder: K-quants round the sub-block scale product first, then the
 * element product (and the min subtraction); Q6_K evaluates (d*sc)*q;
 * IQ4_XS rounds dl = d*(ls-32) then dl*kv. */
int dequant_row(ggml_type_t t, const void *data, uint64_t ne0, float *y)
{
    const uint64_t be = block_elems(t);
    if (!be || ne0 % be) return -1;
    const uint64_t nb = ne0 / be;
    switch (t) {
    case GGML_F32:
        memcpy(y, data, ne0 * sizeof(float));
        return 0;
    case GGML_F16:
        for (uint64_t i = 0; i < ne0; i++) y[i] = fp16_to_f32(((const fp16_t *)data)[i]);
        return 0;
    case GGML_Q8_0: {
        const block_q8_0 *b = data;
        for (uint64_t i = 0; i < nb; i++) {
            const float d = fp16_to_f32(b[i].d);
            for (int l = 0; l < QK8_0; l++) *y++ = d * (float)b[i].qs[l];
        }
        return 0;
    }
    case GGML_Q4_K:
    case GGML_Q5_K: {
        const int five = (t == GGML_Q5_K);
        const uint8_t *p = data;
        const size_t bs = five ? sizeof(block_q5_K) : sizeof(block_q4_K);
        for (uint64_t i = 0; i < nb; i++, p += bs) {
            fp16_t dh, mh;
            memcpy(&dh, p, 2);
            memcpy(&mh, p + 2, 2);
            const float d = fp16_to_f32(dh), dmin = fp16_to_f32(mh);
            const uint8_t *sc = p + 4, *qh = p + 16, *qs = p + (five ? 48 : 16);
            for (int g = 0; g < 4; g++) {
                for (int half = 0; half < 2; half++) {
                    uint8_t s, m;
                    get_scale_min_k4(2 * g + half, sc, &s, &m);
                    const float dd = d * s, mm = dmin * m;
                    for (int l = 0; l < 32; l++) {
                        int q = half ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 15);
                        if (five && ((qh[l] >> (2 * g + half)) & 1)) q += 16;
                        *y++ = dd * q - mm;
                    }
                }
            }
        }
        return 0;
    }
    case GGML_Q6_K: {
        const block_q6_K *b = data;
        for (uint64_t i = 0; i < nb; i++) {
            const float d = fp16_to_f32(b[i].d);
            for (int half = 0; half < 2; half++) {
                const uint8_t *ql = b[i].ql + 64 * half, *qh = b[i].qh + 32 * half;
                const int8_t *sc = b[i].scales + 8 * half;
                for (int quad = 0; quad < 4; quad++)          /* elements 32*quad .. +31 */
                    for (int l = 0; l < 32; l++) {
                        const uint8_t lo = (quad & 1) ? ql[l + 32] : ql[l];
                        const int nib = (quad & 2) ? (lo >> 4) : (lo & 15);
                        const int q = (nib | (((qh[l] >> (2 * quad)) & 3) << 4)) - 32;
                        y[128 * half + 32 * quad + l] = d * sc[l / 16 + 2 * quad] * q;
                    }
            }
            y += QK_K;
        }
        return 0;
    }
    case GGML_IQ4_XS: {
        const block_iq4_xs *b = data;
        for (uint64_t i = 0; i < nb; i++) {
            const float d = fp16_to_f32(b[i].d);
            for (int ib = 0; ib < 8; ib++) {
                const int ls = ((b[i].scales_l[ib >> 1] >> (4 * (ib & 1))) & 15) |
                               (((b[i].scales_h >> (2 * ib)) & 3) << 4);
                const float dl = d * (float)(ls - 32);
                const uint8_t *qs = b[i].qs + 16 * ib;
                for (int j = 0; j < 16; j++) {
                    y[32 * ib + j] = dl * (float)kvalues_iq4nl[qs[j] & 15];
                    y[32 * ib + j + 16] = dl * (float)kvalues_iq4nl[qs[j] >> 4];
                }
            }
            y += QK_K;
        }
        return 0;
    }
    default:
        return -1;
    }
}
