/*
 * or_sample.c -- CPU restatement of the reference sampler (src/sampler.c) and of
 * the non-speculative generation loop (src/main.c:232-248).
 *
 * TEST INFRASTRUCTURE (see oracle.h).  The steps follow the reference so that
 * the chosen token and the generator state are identical for the same inputs:
 * the same xorshift64 generator, the same K-element min-heap selection (the
 * candidate set and its array order, which the tie order of the sort depends
 * on), the C library's qsort with the same comparison, the float/double
 * arithmetic of the softmax, the top-p cut and the draw.
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>

/* sampler.c:8-15 */
static uint64_t rng_next(uint64_t *state)
{
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return *state = x;
}

typedef struct {
    float p;
    uint32_t id;
} cand_t;

/* sampler.c:22-28: descending by value, equal values compare equal */
static int cand_desc(const void *a, const void *b)
{
    const float pa = ((const cand_t *)a)->p, pb = ((const cand_t *)b)->p;
    return pa < pb ? 1 : pa > pb ? -1 : 0;
}

/* sampler.c:30-44: restore the min-heap property below node i */
static void heap_down(cand_t *h, uint32_t n, uint32_t i)
{
    for (;;) {
        const uint32_t l = 2 * i + 1, r = l + 1;
        uint32_t m = i;
        if (l >= n) break;
        if (h[l].p < h[m].p) m = l;
        if (r < n && h[r].p < h[m].p) m = r;
        if (m == i) break;
        const cand_t t = h[i];
        h[i] = h[m];
        h[m] = t;
        i = m;
    }
}

/* sampler.c:46-56 */
void or_sampler_init(or_sampler_t *s, float temp, float top_p, uint32_t top_k, float repeat_penalty, uint64_t seed)
{
    s->temp = temp;
    s->top_p = top_p;
    s->top_k = top_k ? top_k : 40;
    s->repeat_penalty = repeat_penalty > 0.0f ? repeat_penalty : 1.0f;
    s->repeat_last_n = 64;
    s->rng_state = seed ? seed : 0x123456789abcdefULL;
}

/* sampler.c:62-162.  Modifies logits in place (the repeat penalty), as the reference does. */
uint32_t or_sampler_sample(or_sampler_t *s, float *logits, uint32_t V, const uint32_t *tokens, size_t n_tokens)
{
    if (!s || !logits || !V) return 0;
    /* repeat penalty over the last repeat_last_n tokens, once per occurrence (sampler.c:65-77) */
    if (s->repeat_penalty != 1.0f && tokens && n_tokens) {
        for (size_t i = n_tokens > s->repeat_last_n ? n_tokens - s->repeat_last_n : 0; i < n_tokens; i++) {
            const uint32_t t = tokens[i];
            if (t >= V) continue;
            logits[t] = logits[t] > 0.0f ? logits[t] / s->repeat_penalty : logits[t] * s->repeat_penalty;
        }
    }
    /* greedy: first maximum under strict > (sampler.c:79-89) */
    if (s->temp <= 0.0f || s->top_k == 1) {
        uint32_t best = 0;
        for (uint32_t i = 1; i < V; i++)
            if (logits[i] > logits[best]) best = i;
        return best;
    }
    /* top K (<= 256) by a min-heap over the logits in index order (sampler.c:91-119) */
    uint32_t K = s->top_k < 256 ? s->top_k : 256;
    if (K > V) K = V;
    cand_t h[256];
    uint32_t n = 0;
    for (uint32_t i = 0; i < V; i++) {
        const float v = logits[i];
        if (n < K) {
            uint32_t c = n++;
            h[c].p = v;
            h[c].id = i;
            while (c) {
                const uint32_t par = (c - 1) / 2;
                if (!(h[c].p < h[par].p)) break;
                const cand_t t = h[c];
                h[c] = h[par];
                h[par] = t;
                c = par;
            }
        } else if (v > h[0].p) {
            h[0].p = v;
            h[0].id = i;
            heap_down(h, K, 0);
        }
    }
    qsort(h, K, sizeof(cand_t), cand_desc);
    /* softmax at temperature: float exponentials, double sum (sampler.c:123-133) */
    const float top = h[0].p / s->temp;
    double sum = 0.0;
    for (uint32_t i = 0; i < K; i++) {
        h[i].p = expf(h[i].p / s->temp - top);
        sum += h[i].p;
    }
    const float inv = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
    for (uint32_t i = 0; i < K; i++) h[i].p *= inv;
    /* nucleus: the shortest prefix whose float running sum reaches top_p (sampler.c:135-145) */
    uint32_t nc = K;
    if (s->top_p < 1.0f) {
        float c = 0.0f;
        uint32_t i = 0;
        for (; i < K; i++) {
            c += h[i].p;
            if (c >= s->top_p) break;
        }
        nc = (i < K ? i : K - 1) + 1;
    }
    float tot = 0.0f;
    for (uint32_t i = 0; i < nc; i++) tot += h[i].p;
    /* draw (sampler.c:152-161) */
    const float r = ((float)(rng_next(&s->rng_state) % 10000000) / 10000000.0f) * tot;
    float acc = 0.0f;
    for (uint32_t i = 0; i < nc; i++) {
        acc += h[i].p;
        if (acc >= r) return h[i].id;
    }
    return h[0].id;
}
