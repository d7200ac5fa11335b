/*
 * or_quant.c -- oracle restatement of the reference quant formats
 * (reference include/quant.h:14-68, src/quant.c:6-208).
 * Test infrastructure only (see oracle.h).
 */
#include "oracle.h"
#include <string.h>

/* quant.c:6-28 : portable fp16 -> fp32 including subnormal renormalisation */
float or_fp16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {                 /* subnormal: shift the mantissa up to the hidden bit */
            int ex = 113;        /* 127 - 15 + 1 */
            while (!(m & 0x400u)) { m <<= 1; ex--; }
            bits = sign | ((uint32_t)ex << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* quant.c:30-32 : IQ4_NL non-linear codebook */
const int8_t or_iq4nl_values[16] = {
    -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };

size_t or_block_bytes(int t)               /* quant.c:34-45 ; quant.h:15-68 sizes */
{
    switch (t) {
    case OR_F32: return 4;   case OR_F16: return 2;
    case OR_Q8_0: return 34; case OR_Q4_K: return 144; case OR_Q5_K: return 176;
    case OR_Q6_K: return 210; case OR_IQ4_XS: return 136;
    default: return 0;
    }
}

size_t or_block_elems(int t)               /* quant.c:48-59 */
{
    switch (t) {
    case OR_F32: case OR_F16: return 1;
    case OR_Q8_0: return 32;
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_IQ4_XS: return 256;
    default: return 0;
    }
}

size_t or_row_bytes(int t, uint64_t ne0)   /* quant.c:61-65 */
{
    size_t be = or_block_elems(t);
    return be ? (size_t)(ne0 / be) * or_block_bytes(t) : 0;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* quant.h:21-29 : packed 6-bit scale/min pair j of a Q4_K/Q5_K block */
void or_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quant.c:86-92 */
static void dq_q8_0(const uint8_t *b, float *y, uint64_t nb)
{
    for (uint64_t i = 0; i < nb; i++, b += 34) {
        const float d = or_fp16_to_f32(rd16(b));
        for (int l = 0; l < 32; l++) y[i * 32 + l] = d * (float)(int8_t)b[2 + l];
    }
}

/* quant.c:94-112 (two roundings: d*sc, then *q - m) */
static void dq_q4_K(const uint8_t *b, float *y, uint64_t nb)
{
    for (uint64_t i = 0; i < nb; i++, b += 144) {
        const float d = or_fp16_to_f32(rd16(b)), dm = or_fp16_to_f32(rd16(b + 2));
        const uint8_t *sc = b + 4, *q = b + 16;
        for (int g = 0; g < 4; g++, q += 32) {
            uint8_t s, m;
            or_scale_min_k4(2 * g, sc, &s, &m);
            const float d1 = d * s, m1 = dm * m;
            or_scale_min_k4(2 * g + 1, sc, &s, &m);
            const float d2 = d * s, m2 = dm * m;
            for (int l = 0; l < 32; l++) *y++ = d1 * (q[l] & 15) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (q[l] >> 4) - m2;
        }
    }
}

/* quant.c:114-138 */
static void dq_q5_K(const uint8_t *b, float *y, uint64_t nb)
{
    for (uint64_t i = 0; i < nb; i++, b += 176) {
        const float d = or_fp16_to_f32(rd16(b)), dm = or_fp16_to_f32(rd16(b + 2));
        const uint8_t *sc = b + 4, *qh = b + 16, *q = b + 48;
        for (int g = 0; g < 4; g++, q += 32) {
            uint8_t s, m;
            or_scale_min_k4(2 * g, sc, &s, &m);
            const float d1 = d * s, m1 = dm * m;
            or_scale_min_k4(2 * g + 1, sc, &s, &m);
            const float d2 = d * s, m2 = dm * m;
            for (int l = 0; l < 32; l++)
                *y++ = d1 * ((q[l] & 15) + ((qh[l] >> (2 * g)) & 1 ? 16 : 0)) - m1;
            for (int l = 0; l < 32; l++)
                *y++ = d2 * ((q[l] >> 4) + ((qh[l] >> (2 * g + 1)) & 1 ? 16 : 0)) - m2;
        }
    }
}

/* quant.c:140-164 : value = (d * sc) * q, evaluated left to right */
static void dq_q6_K(const uint8_t *b, float *y, uint64_t nb)
{
    for (uint64_t i = 0; i < nb; i++, b += 210) {
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        const float d = or_fp16_to_f32(rd16(b + 208));
        for (int h = 0; h < 2; h++, y += 128, ql += 64, qh += 32, sc += 8) {
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l]      = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
        }
    }
}

/* quant.c:166-182 : dl = d * (ls - 32) rounded, then dl * kv rounded */
static void dq_iq4_xs(const uint8_t *b, float *y, uint64_t nb)
{
    for (uint64_t i = 0; i < nb; i++, b += 136) {
        const float d = or_fp16_to_f32(rd16(b));
        const uint16_t sh = rd16(b + 2);
        const uint8_t *sl = b + 4, *qs = b + 8;
        for (int ib = 0; ib < 8; ib++, y += 32, qs += 16) {
            const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
            const float dl = d * (float)(ls - 32);
            for (int j = 0; j < 16; j++) {
                y[j]      = dl * (float)or_iq4nl_values[qs[j] & 15];
                y[j + 16] = dl * (float)or_iq4nl_values[qs[j] >> 4];
            }
        }
    }
}

/* quant.c:184-208 */
int or_dequant_row(int t, const void *data, uint64_t ne0, float *dst)
{
    const size_t be = or_block_elems(t);
    if (!be || ne0 % be) return -1;
    const uint64_t nb = ne0 / be;
    const uint8_t *b = (const uint8_t *)data;
    switch (t) {
    case OR_F32: memcpy(dst, data, ne0 * 4); break;
    case OR_F16: for (uint64_t i = 0; i < ne0; i++) dst[i] = or_fp16_to_f32(rd16(b + 2 * i)); break;
    case OR_Q8_0: dq_q8_0(b, dst, nb); break;
    case OR_Q4_K: dq_q4_K(b, dst, nb); break;
    case OR_Q5_K: dq_q5_K(b, dst, nb); break;
    case OR_Q6_K: dq_q6_K(b, dst, nb); break;
    case OR_IQ4_XS: dq_iq4_xs(b, dst, nb); break;
    default: return -1;
    }
    return 0;
}
