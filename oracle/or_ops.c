/*
 * or_ops.c -- oracle restatement of the reference elementwise / norm ops
 * (reference src/kernels.c:741-939) and greedy argmax (src/model.c:746-756).
 * 8-lane AVX2 loops are emulated lane by lane; scalar tails use libm exactly
 * like the reference.  Test infrastructure only.
 */
#include "oracle.h"
#include <math.h>
#include <string.h>

static float hsum8(const float *v)          /* kernels.c:15-24 */
{
    const float L0 = v[0] + v[4], L1 = v[1] + v[5], L2 = v[2] + v[6], L3 = v[3] + v[7];
    return (L0 + L1) + (L2 + L3);
}

/* 8-lane sum of squares with FMA, then scalar tail without contraction
 * (kernels.c:742-751 and :781-790) */
static float sumsq(const float *x, uint64_t n)
{
    float acc[8] = {0};
    uint64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
    float s = hsum8(acc);
    for (; i < n; i++) s += x[i] * x[i];
    return s;
}

/* kernels.c:741-777 */
void or_rmsnorm(float *out, const float *x, const float *w, uint64_t n, float eps)
{
    const float ss = sumsq(x, n);
    const float mean = ss / (float)n;
    const float scale = 1.0f / sqrtf(mean + eps);
    for (uint64_t i = 0; i < n; i++) out[i] = w ? (x[i] * scale) * w[i] : x[i] * scale;
}

/* kernels.c:780-805 */
void or_l2norm(float *out, const float *x, uint64_t n, float eps)
{
    const float nrm = sqrtf(sumsq(x, n));
    const float scale = 1.0f / (nrm > eps ? nrm : eps);
    for (uint64_t i = 0; i < n; i++) out[i] = x[i] * scale;
}

/* kernels.c:807-822 exp256_ps, one lane: clamp to [-88,88], k = rint(x*log2e),
 * r = x - k*ln2 (single rounding), degree-7 Taylor polynomial in Horner form,
 * times 2^k built from the exponent bits. */
float or_exp8_lane(float x)
{
    float xc = (x < 88.0f) ? x : 88.0f;              /* _mm256_min_ps(x, 88)  */
    xc = (xc > -88.0f) ? xc : -88.0f;                /* _mm256_max_ps(., -88) */
    const float k = rintf(xc * 1.4426950408889634f);
    const float r = fmaf(-k, 0.6931471805599453f, xc);
    float p = 0.000198412698f;
    p = fmaf(p, r, 0.00139304842f);
    p = fmaf(p, r, 0.00833333333f);
    p = fmaf(p, r, 0.04166666666f);
    p = fmaf(p, r, 0.16666666666f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const uint32_t bits = (uint32_t)((int32_t)k + 127) << 23;
    float s;
    memcpy(&s, &bits, 4);
    return p * s;
}

/* kernels.c:825-847 */
void or_silu_inplace(float *x, uint64_t n)
{
    uint64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            const float v = x[i + l];
            const float sig = 1.0f / (1.0f + or_exp8_lane(0.0f - v));
            x[i + l] = v * sig;
        }
    for (; i < n; i++) {
        const float v = x[i];
        if (v < -20.0f) x[i] = v * expf(v);
        else if (v > 20.0f) x[i] = v;
        else x[i] = v / (1.0f + expf(-v));
    }
}

/* kernels.c:850-871 */
void or_sigmoid_inplace(float *x, uint64_t n)
{
    uint64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++)
            x[i + l] = 1.0f / (1.0f + or_exp8_lane(0.0f - x[i + l]));
    for (; i < n; i++) {
        const float v = x[i];
        if (v < -20.0f) x[i] = 0.0f;
        else if (v > 20.0f) x[i] = 1.0f;
        else x[i] = 1.0f / (1.0f + expf(-v));
    }
}

/* kernels.c:874-885 */
void or_softplus_inplace(float *x, uint64_t n)
{
    for (uint64_t i = 0; i < n; i++) {
        const float v = x[i];
        if (v > 30.0f) x[i] = v;
        else if (v < -30.0f) x[i] = expf(v);
        else x[i] = log1pf(expf(v));
    }
}

/* kernels.c:901-939 : vector max, vector exp + 8-lane float sum, double tail sum */
void or_softmax_inplace(float *x, uint64_t n)
{
    if (n == 0) return;
    float vmax[8];
    for (int l = 0; l < 8; l++) vmax[l] = x[0];
    uint64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            const float v = x[i + l];
            vmax[l] = (vmax[l] > v) ? vmax[l] : v;   /* _mm256_max_ps(vmax, v) */
        }
    /* hmax256, kernels.c:890-899 */
    float m0 = vmax[0] > vmax[4] ? vmax[0] : vmax[4], m1 = vmax[1] > vmax[5] ? vmax[1] : vmax[5];
    float m2 = vmax[2] > vmax[6] ? vmax[2] : vmax[6], m3 = vmax[3] > vmax[7] ? vmax[3] : vmax[7];
    float a = m0 > m1 ? m0 : m1, b = m2 > m3 ? m2 : m3;
    float mx = a > b ? a : b;
    for (; i < n; i++) if (x[i] > mx) mx = x[i];

    float vs[8] = {0};
    i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            const float e = or_exp8_lane(x[i + l] - mx);
            x[i + l] = e;
            vs[l] += e;
        }
    double sum = (double)hsum8(vs);
    for (; i < n; i++) {
        const float e = expf(x[i] - mx);
        x[i] = e;
        sum += (double)e;
    }
    const float inv = (float)(1.0 / sum);
    for (i = 0; i < n; i++) x[i] *= inv;
}

/* model.c:746-756 : strict '>' so the lowest index wins ties */
uint32_t or_argmax(const float *logits, uint32_t n)
{
    uint32_t best = 0;
    float mv = logits[0];
    for (uint32_t i = 1; i < n; i++)
        if (logits[i] > mv) { mv = logits[i]; best = i; }
    return best;
}
