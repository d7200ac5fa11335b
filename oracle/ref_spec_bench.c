/*
 * ref_spec_bench.c -- times the reference engine (oracle/_ref/libqwenref.so,
 * compiled from the reference sources) on the greedy MTP speculative-decode
 * loop, for the CPU baseline of the benchmark.  Test/benchmark infrastructure:
 * nothing in the product links it.
 *
 * The loop follows the reference driver's cycle (src/main.c:158-231): k MTP
 * drafts, one batched verify of k+1 tokens with checkpoints, greedy
 * acceptance, rollback of the recurrent states, MTP re-anchor.  The reference
 * keeps SPEC_MAX_B-1 = 2 state checkpoints (include/model.h:113), so with k = 3
 * a cycle that accepts exactly 2 drafts cannot be rolled back by the reference;
 * the run then stops and reports -2 (random-init weights accept ~0 drafts).
 *
 * ref_sample_bench times the reference's sampled decode (src/main.c:232-248):
 * sampler_sample over the prompt and the generated tokens, then model_forward.
 */
#define _POSIX_C_SOURCE 200809L
#include "model.h"
#include "sampler.h"
#include "threadpool.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double wall(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* out[0] = prefill seconds, out[1] = timed seconds, out[2] = tokens emitted in
 * the timed cycles, out[3] = timed cycles, out[4] = drafts accepted.
 * Returns 0, -1 (load failure) or -2 (acceptance depth without checkpoint). */
int ref_spec_bench(const char *gguf, uint32_t n_ctx, const uint32_t *prompt, uint32_t n_prompt, uint32_t k,
                   uint32_t warm_cycles, uint32_t max_cycles, double max_secs, int threads, double *out)
{
    qwen_model_t *m = calloc(1, sizeof *m);
    if (!m || model_init(m, gguf, n_ctx)) { free(m); return -1; }
    pool_t *pool = pool_create(threads, 1);
    const uint32_t V = m->cfg.vocab_size, E = m->dims.n_embd;
    int rc = 0;
    double t = wall();
    for (uint32_t p = 0, B; p < n_prompt; p += B) {
        B = n_prompt - p < PREFILL_MAX_B ? n_prompt - p : PREFILL_MAX_B;
        model_forward_batch(m, pool, prompt + p, p, B, 0);
        mtp_forward_batch(m, pool, prompt + p, p, B, 0);
    }
    const float *last = m->logits_b + (size_t)((n_prompt - 1) % PREFILL_MAX_B) * V;
    out[0] = wall() - t;
    double t_start = 0.0;
    uint64_t toks = 0, cyc = 0, acc = 0;
    for (uint32_t c = 0; c < warm_cycles + max_cycles; c++) {
        if (c == warm_cycles) { t_start = wall(); toks = cyc = acc = 0; }
        if (c > warm_cycles && wall() - t_start > max_secs) break;
        const uint32_t P = m->pos - 1;
        if (P + k + 2 >= n_ctx) break;
        uint32_t cand[16];
        cand[0] = model_sample_greedy(last, V);
        for (uint32_t s = 1; s <= k; s++) {
            mtp_forward(m, pool, cand[s - 1], P + s, 1);
            cand[s] = model_sample_greedy(m->logits, V);
        }
        model_forward_batch(m, pool, cand, P + 1, k + 1, 1);
        uint32_t j = k;
        for (uint32_t i = 0; i < k; i++)
            if (model_sample_greedy(m->logits_b + (size_t)i * V, V) != cand[i + 1]) { j = i; break; }
        if (j < k && j + 1 >= SPEC_MAX_B) { rc = -2; break; }
        toks += j + 1;
        acc += j;
        cyc++;
        if (j < k) {
            model_rollback_to(m, j);
            m->pos = P + j + 2;
        }
        memcpy(m->mtp_h, m->h_save + (size_t)j * E, E * sizeof(float));
        mtp_forward(m, pool, cand[j], P + j + 1, 0);
        last = m->logits_b + (size_t)j * V;
    }
    out[1] = wall() - t_start;
    out[2] = (double)toks;
    out[3] = (double)cyc;
    out[4] = (double)acc;
    pool_destroy(pool);
    model_free(m);
    free(m);
    return rc;
}

/* out[0] = prefill seconds, out[1] = timed decode seconds, out[2] = tokens sampled in it,
 * out[3] = seconds inside sampler_sample, out[4] = sampler_sample calls.  Returns 0 or -1. */
int ref_sample_bench(const char *gguf, uint32_t n_ctx, const uint32_t *prompt, uint32_t n_prompt, float temp,
                     float top_p, uint32_t top_k, float repeat_penalty, uint64_t seed, uint32_t max_tokens,
                     double max_secs, int threads, double *out)
{
    qwen_model_t *m = calloc(1, sizeof *m);
    if (!m || model_init(m, gguf, n_ctx)) { free(m); return -1; }
    pool_t *pool = pool_create(threads, 1);
    sampler_t *smp = sampler_init(temp, top_p, top_k, repeat_penalty, seed);
    uint32_t *all = malloc(sizeof(uint32_t) * ((size_t)n_prompt + max_tokens + 1));
    const uint32_t V = m->cfg.vocab_size;
    double t = wall();
    for (uint32_t p = 0, B; p < n_prompt; p += B) {
        B = n_prompt - p < PREFILL_MAX_B ? n_prompt - p : PREFILL_MAX_B;
        model_forward_batch(m, pool, prompt + p, p, B, 0);
    }
    float *lg = m->logits_b + (size_t)((n_prompt - 1) % PREFILL_MAX_B) * V;
    out[0] = wall() - t;
    memcpy(all, prompt, sizeof(uint32_t) * n_prompt);
    size_t n_all = n_prompt;
    double t_smp = 0.0;
    uint32_t gen = 0;
    const double t_start = wall();
    for (;;) {
        const double t1 = wall();
        const uint32_t cur = sampler_sample(smp, lg, V, all, n_all);
        t_smp += wall() - t1;
        all[n_all++] = cur;
        gen++;
        if (gen >= max_tokens || m->pos >= n_ctx || wall() - t_start > max_secs) break;
        model_forward(m, pool, cur, m->pos);
        lg = m->logits;
    }
    out[1] = wall() - t_start;
    out[2] = (double)gen;
    out[3] = t_smp;
    out[4] = (double)gen;
    free(all);
    sampler_free(smp);
    pool_destroy(pool);
    model_free(m);
    free(m);
    return 0;
}
