/*
 * or_gemv.c -- oracle restatement of the reference batched dequant-GEMV
 * (reference src/kernels.c:15-37, 123-131, 298-599, 632-648).
 *
 * The reference accumulates every row in two 8-lane AVX2 accumulators
 * (acc0/acc1) with FMA and reduces them with hsum256_2.  Here each lane is a
 * scalar float and every _mm256_fmadd_ps is one fmaf() per lane, so the fp32
 * result is bit-identical to the reference's.  Test infrastructure only.
 */
#include "oracle.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define MAXB 8
extern const int8_t or_iq4nl_values[16];
void or_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn);

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

typedef struct { float v[8]; } lane8;

/* kernels.c:15-28 hsum256 / hsum256_2 : ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) */
static float hsum8(const lane8 *a)
{
    const float L0 = a->v[0] + a->v[4], L1 = a->v[1] + a->v[5];
    const float L2 = a->v[2] + a->v[6], L3 = a->v[3] + a->v[7];
    return (L0 + L1) + (L2 + L3);
}
static float hsum8_2(const lane8 *a, const lane8 *b)
{
    lane8 s;
    for (int l = 0; l < 8; l++) s.v[l] = a->v[l] + b->v[l];
    return hsum8(&s);
}

/* kernels.c:330-340 fmadd16_i8_n : w = (float)q * ds (rounded), then one FMA
 * per lane; elements 0..7 go to lanes 0..7, then elements 8..15 again. */
static void fma16(const int *q, float ds, const float *x, uint64_t ldx, int n,
                  lane8 *acc, uint64_t off)
{
    for (int half = 0; half < 2; half++) {
        float w[8];
        for (int l = 0; l < 8; l++) w[l] = (float)q[8 * half + l] * ds;
        for (int t = 0; t < n; t++) {
            const float *xp = x + t * ldx + off + 8 * half;
            for (int l = 0; l < 8; l++) acc[t].v[l] = fmaf(w[l], xp[l], acc[t].v[l]);
        }
    }
}

/* kernels.c:123-131 xsums32 : per-32 sums, lane l = (x[l]+x[8+l]) + (x[16+l]+x[24+l]) */
static void xsums32(const float *x, uint64_t n32, float *xs)
{
    for (uint64_t k = 0; k < n32; k++) {
        lane8 s;
        const float *p = x + 32 * k;
        for (int l = 0; l < 8; l++) s.v[l] = (p[l] + p[8 + l]) + (p[16 + l] + p[24 + l]);
        xs[k] = hsum8(&s);
    }
}

/* kernels.c:342-357 dot_f32_b */
static void dot_f32(const float *w, const float *x, uint64_t ldx, int n, float *out,
                    uint64_t ldo, uint64_t r, uint64_t len)
{
    lane8 acc[MAXB];
    memset(acc, 0, sizeof acc);
    uint64_t i = 0;
    for (; i + 8 <= len; i += 8)
        for (int t = 0; t < n; t++)
            for (int l = 0; l < 8; l++)
                acc[t].v[l] = fmaf(w[i + l], x[t * ldx + i + l], acc[t].v[l]);
    const uint64_t tail = len & ~(uint64_t)7;
    for (int t = 0; t < n; t++) {
        float s = hsum8(&acc[t]);
        for (uint64_t k = tail; k < len; k++) s += w[k] * x[t * ldx + k];
        out[t * ldo + r] = s;
    }
}

/* kernels.c:359-371 dot_q8_0_b */
static void dot_q8_0(const uint8_t *b, size_t nb, const float *x, uint64_t ldx, int n,
                     float *out, uint64_t ldo, uint64_t r)
{
    lane8 a0[MAXB], a1[MAXB];
    memset(a0, 0, sizeof a0); memset(a1, 0, sizeof a1);
    int q[16];
    for (size_t i = 0; i < nb; i++, b += 34) {
        const float d = or_fp16_to_f32(rd16(b));
        for (int l = 0; l < 16; l++) q[l] = (int8_t)b[2 + l];
        fma16(q, d, x, ldx, n, a0, i * 32);
        for (int l = 0; l < 16; l++) q[l] = (int8_t)b[18 + l];
        fma16(q, d, x, ldx, n, a1, i * 32 + 16);
    }
    for (int t = 0; t < n; t++) out[t * ldo + r] = hsum8_2(&a0[t], &a1[t]);
}

/* kernels.c:373-412 dot_iq4_xs_b : even sub-blocks -> acc0, odd -> acc1 */
static void dot_iq4_xs(const uint8_t *b, size_t nb, const float *x, uint64_t ldx, int n,
                       float *out, uint64_t ldo, uint64_t r)
{
    lane8 acc[2][MAXB];
    memset(acc, 0, sizeof acc);
    int q[16];
    for (size_t i = 0; i < nb; i++, b += 136) {
        const float d = or_fp16_to_f32(rd16(b));
        const uint16_t sh = rd16(b + 2);
        const uint8_t *sl = b + 4, *qs = b + 8;
        for (int ib = 0; ib < 8; ib++) {
            const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
            const float dl = d * (float)(ls - 32);
            const uint8_t *by = qs + 16 * ib;
            for (int l = 0; l < 16; l++) q[l] = or_iq4nl_values[by[l] & 15];
            fma16(q, dl, x, ldx, n, acc[ib & 1], i * 256 + ib * 32);
            for (int l = 0; l < 16; l++) q[l] = or_iq4nl_values[by[l] >> 4];
            fma16(q, dl, x, ldx, n, acc[ib & 1], i * 256 + ib * 32 + 16);
        }
    }
    for (int t = 0; t < n; t++) out[t * ldo + r] = hsum8_2(&acc[0][t], &acc[1][t]);
}

/* kernels.c:414-510 dot_q4_K_b / dot_q5_K_b (hb = 1 for Q5_K) */
static void dot_qk_45(const uint8_t *b, size_t nb, int q5, const float *x, uint64_t ldx,
                      const float *xs, int n, float *out, uint64_t ldo, uint64_t r)
{
    lane8 a0[MAXB], a1[MAXB];
    float accm[MAXB];
    memset(a0, 0, sizeof a0); memset(a1, 0, sizeof a1); memset(accm, 0, sizeof accm);
    const size_t bs = q5 ? 176 : 144;
    int q[16];
    for (size_t i = 0; i < nb; i++, b += bs) {
        const float d = or_fp16_to_f32(rd16(b)), dm = or_fp16_to_f32(rd16(b + 2));
        const uint8_t *scl = b + 4, *qh = b + 16, *qsb = b + (q5 ? 48 : 16);
        for (int g = 0; g < 4; g++) {
            uint8_t sc, m;
            or_scale_min_k4(2 * g, scl, &sc, &m);
            const float d1 = d * sc, m1 = dm * m;
            or_scale_min_k4(2 * g + 1, scl, &sc, &m);
            const float d2 = d * sc, m2 = dm * m;
            const uint64_t base = i * 256 + g * 64;
            const uint8_t *qs = qsb + 32 * g;
            for (int part = 0; part < 2; part++) {          /* bytes 0..15, 16..31 */
                for (int l = 0; l < 16; l++) {
                    const int li = 16 * part + l;
                    q[l] = (qs[li] & 15) + (q5 ? (((qh[li] >> (2 * g)) & 1) << 4) : 0);
                }
                fma16(q, d1, x, ldx, n, a0, base + 16 * part);
            }
            for (int part = 0; part < 2; part++) {
                for (int l = 0; l < 16; l++) {
                    const int li = 16 * part + l;
                    q[l] = (qs[li] >> 4) + (q5 ? (((qh[li] >> (2 * g + 1)) & 1) << 4) : 0);
                }
                fma16(q, d2, x, ldx, n, a1, base + 32 + 16 * part);
            }
            for (int t = 0; t < n; t++)
                accm[t] += m1 * xs[t * (nb * 8) + i * 8 + 2 * g]
                         + m2 * xs[t * (nb * 8) + i * 8 + 2 * g + 1];
        }
    }
    for (int t = 0; t < n; t++) out[t * ldo + r] = hsum8_2(&a0[t], &a1[t]) - accm[t];
}

/* kernels.c:512-565 dot_q6_K_b */
static void dot_q6_K(const uint8_t *b, size_t nb, const float *x, uint64_t ldx, int n,
                     float *out, uint64_t ldo, uint64_t r)
{
    lane8 a0[MAXB], a1[MAXB];
    memset(a0, 0, sizeof a0); memset(a1, 0, sizeof a1);
    int q[16];
    for (size_t i = 0; i < nb; i++, b += 210) {
        const float d = or_fp16_to_f32(rd16(b + 208));
        for (int nn = 0; nn < 2; nn++) {
            const uint8_t *ql = b + nn * 64, *qh = b + 128 + nn * 32;
            const int8_t *sc = (const int8_t *)(b + 192 + nn * 8);
            const uint64_t base = i * 256 + nn * 128;
            for (int hh = 0; hh < 2; hh++) {
                const uint8_t *l1 = ql + 16 * hh, *l2 = ql + 16 * (hh + 2), *h1 = qh + 16 * hh;
                const uint64_t xb = base + hh * 16;
                for (int l = 0; l < 16; l++) q[l] = ((l1[l] & 15) | ((h1[l] & 3) << 4)) - 32;
                fma16(q, d * sc[hh + 0], x, ldx, n, a0, xb);
                for (int l = 0; l < 16; l++) q[l] = ((l2[l] & 15) | (((h1[l] >> 2) & 3) << 4)) - 32;
                fma16(q, d * sc[hh + 2], x, ldx, n, a1, xb + 32);
                for (int l = 0; l < 16; l++) q[l] = ((l1[l] >> 4) | (((h1[l] >> 4) & 3) << 4)) - 32;
                fma16(q, d * sc[hh + 4], x, ldx, n, a0, xb + 64);
                for (int l = 0; l < 16; l++) q[l] = ((l2[l] >> 4) | (((h1[l] >> 6) & 3) << 4)) - 32;
                fma16(q, d * sc[hh + 6], x, ldx, n, a1, xb + 96);
            }
        }
    }
    for (int t = 0; t < n; t++) out[t * ldo + r] = hsum8_2(&a0[t], &a1[t]);
}

/* kernels.c:570-599 gemv_rows_batch (unsupported types write zeros, :596) */
void or_gemv_rows_batch(int type, const void *W, uint64_t ne0, const float *x, uint64_t ldx,
                        int n, float *out, uint64_t ldo, uint64_t r0, uint64_t r1)
{
    const size_t rb = or_row_bytes(type, ne0);
    const size_t nb = (type == OR_Q8_0) ? ne0 / 32 : ne0 / 256;
    float *xs = NULL;
    if (type == OR_Q4_K || type == OR_Q5_K) {
        xs = (float *)malloc(sizeof(float) * (size_t)n * (ne0 / 32));
        for (int t = 0; t < n; t++) xsums32(x + t * ldx, ne0 / 32, xs + t * (ne0 / 32));
    }
    for (uint64_t r = r0; r < r1; r++) {
        const uint8_t *row = (const uint8_t *)W + r * rb;
        switch (type) {
        case OR_F32:    dot_f32((const float *)row, x, ldx, n, out, ldo, r, ne0); break;
        case OR_Q8_0:   dot_q8_0(row, nb, x, ldx, n, out, ldo, r); break;
        case OR_IQ4_XS: dot_iq4_xs(row, nb, x, ldx, n, out, ldo, r); break;
        case OR_Q4_K:   dot_qk_45(row, nb, 0, x, ldx, xs, n, out, ldo, r); break;
        case OR_Q5_K:   dot_qk_45(row, nb, 1, x, ldx, xs, n, out, ldo, r); break;
        case OR_Q6_K:   dot_q6_K(row, nb, x, ldx, n, out, ldo, r); break;
        default: for (int t = 0; t < n; t++) out[t * ldo + r] = 0.0f; break;
        }
    }
    free(xs);
}

typedef struct {
    int type; const void *W; uint64_t ne0, ne1; const float *x; uint64_t ldx; int n;
    float *out; uint64_t ldo; int tid, nt;
} gemv_job;

static void *gemv_worker(void *p)
{
    gemv_job *j = (gemv_job *)p;
    const uint64_t r0 = j->ne1 * (uint64_t)j->tid / j->nt, r1 = j->ne1 * (uint64_t)(j->tid + 1) / j->nt;
    or_gemv_rows_batch(j->type, j->W, j->ne0, j->x, j->ldx, j->n, j->out, j->ldo, r0, r1);
    return NULL;
}

/* kernels.c:632-648 : contiguous row ranges per thread (bits do not depend on the split) */
void or_gemv_batch(int type, const void *W, uint64_t ne0, uint64_t ne1, const float *x,
                   uint64_t ldx, int n, float *out, uint64_t ldo, int n_threads)
{
    if (n_threads <= 1 || ne1 < 64) {
        or_gemv_rows_batch(type, W, ne0, x, ldx, n, out, ldo, 0, ne1);
        return;
    }
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    gemv_job jobs[64];
    for (int k = 0; k < n_threads; k++) {
        jobs[k] = (gemv_job){ type, W, ne0, ne1, x, ldx, n, out, ldo, k, n_threads };
        pthread_create(&th[k], NULL, gemv_worker, &jobs[k]);
    }
    for (int k = 0; k < n_threads; k++) pthread_join(th[k], NULL);
}
