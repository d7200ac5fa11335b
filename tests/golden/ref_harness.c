/*
 * ref_harness.c -- drives the compiled reference engine (oracle/_ref) through
 * its public API to produce golden vectors.  Built and run only where the
 * reference checkout exists (by make_golden.py); its outputs are committed
 * as fixtures next to this file.
 *
 * usage: ref_harness <model.gguf> <out_dir> <n_ctx>
 *        ref_harness <model.gguf> <out_dir> <n_ctx> greedy <prompt.u32> <n_gen>
 *        ref_harness <model.gguf> <out_dir> <n_ctx> spec <n_prompt> <n_predict>
 *        ref_harness <model.gguf> <out_dir> <n_ctx> long <n_prompt> <n_predict>
 * The spec form runs every speculative scenario from a prefill of n_prompt ids
 * and writes, per scenario, the stream (.u32), j per cycle (_j.u32), the logits
 * the next cycle would start from (_last.f32) and the final MTP hidden state
 * (_mtph.f32): spec_k{1,2} (main.c's batched loop), spec_seq_k{1..7}
 * (sequential verification, any k), spec_f{1,2}_k{1..7} (forced acceptance,
 * sequential verification), and greedy.u32 (n_predict + 8 tokens: the tokens a
 * cycle cut by n_predict verified and kept are on it too).  The long form
 * (a prompt that fills most of n_ctx) writes prefill_last.f32 and only
 * spec_seq_k / spec_f1_k for k = 1, 3, 5, 7.
 * The second form (full-size model) prefills the prompt in chunks of 8 and
 * decodes n_gen tokens greedily with model_forward, writing
 *   stream.u32        the greedy tokens
 *   gap.f32           top-1 minus top-2 logit of the logits each token was taken from
 *   prefill_logits.f32 logits of the last prompt token
 * Writes raw little-endian arrays (see make_golden.py for the manifest):
 *   seq_logits.f32      sequential model_forward logits for prompt[0..7]
 *   batch_logits.f32    model_forward_batch(prompt[0..7], pos 0, B=8) logits_b
 *   batch_hsave.f32     matching h_save
 *   mtp_logits.f32      mtp_forward(prompt[8], pos 8, 1) after an 8-token prefill + MTP prefill
 *   rollback_logits.f32 debug_rollback.c pattern: batch(3) -> rollback_to(1) -> batch(3)
 *   spec_k{K}.u32       greedy spec streams (main.c:158-231 loop, batched verify, K=1,2)
 *   spec_seq_k{K}.u32   same streams with sequential verification (any K)
 *   spec_j_k{K}.u32     accepted index j per cycle
 *   greedy.u32          plain greedy stream (argmax of model_forward)
 *   sample_cfg.f64      [4][5] sampler configurations: temp, top_p, top_k, repeat_penalty, seed
 *   sample_c{C}.u32     sampled streams (main.c:232-248: sampler_init + sampler_sample over the prompt
 *                       and the generated tokens), sampler configuration C of SAMPLE_CFG
 */
#define _POSIX_C_SOURCE 200809L
#include "model.h"
#include "sampler.h"
#include "threadpool.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static void dump(const char *dir, const char *name, const void *p, size_t bytes)
{
    char path[512];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(p, 1, bytes, f) != bytes) { perror(path); exit(2); }
    fclose(f);
}

static uint32_t prompt_tok(uint32_t i, uint32_t V) { return (uint32_t)((i * 2654435761u + 12345u) % V); }

/* worker pool of the reference calls (NULL = serial; the long form uses every core:
 * the reference's row and head partitions do not change any result bit) */
static pool_t *g_pool;

/* prefill exactly as main.c:133-152 */
static void prefill(qwen_model_t *m, const uint32_t *p, uint32_t n, int mtp)
{
    uint32_t pos = 0, last = 0;
    while (pos < n) {
        uint32_t B = n - pos > PREFILL_MAX_B ? PREFILL_MAX_B : n - pos;
        model_forward_batch(m, g_pool, p + pos, pos, B, 0);
        if (mtp) mtp_forward_batch(m, g_pool, p + pos, pos, B, 0);
        pos += B;
        last = B;
    }
    memcpy(m->logits, m->logits_b + (size_t)(last - 1) * m->cfg.vocab_size,
           (size_t)m->cfg.vocab_size * sizeof(float));
}

/* top-1 index (lowest on ties, as model_sample_greedy) and top-1 minus top-2 value */
static uint32_t top2(const float *l, uint32_t V, float *gap)
{
    uint32_t b = 0;
    for (uint32_t i = 1; i < V; i++) if (l[i] > l[b]) b = i;
    float second = -3.4e38f;
    for (uint32_t i = 0; i < V; i++) if (i != b && l[i] > second) second = l[i];
    *gap = l[b] - second;
    return b;
}

static int greedy_mode(const char *path, const char *dir, uint32_t n_ctx, const char *prompt_file, uint32_t n_gen)
{
    FILE *f = fopen(prompt_file, "rb");
    if (!f) { perror(prompt_file); return 1; }
    uint32_t prompt[4096];
    const uint32_t n_prompt = (uint32_t)fread(prompt, 4, 4096, f);
    fclose(f);
    qwen_model_t *m = calloc(1, sizeof *m);
    if (!m || model_init(m, path, n_ctx)) return 1;
    const long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
    pool_t *pool = pool_create(ncpu > 0 ? (int)ncpu : 1, 1);
    const uint32_t V = m->cfg.vocab_size;
    uint32_t pos = 0, last = 0;
    while (pos < n_prompt) {
        uint32_t B = n_prompt - pos > PREFILL_MAX_B ? PREFILL_MAX_B : n_prompt - pos;
        model_forward_batch(m, pool, prompt + pos, pos, B, 0);
        pos += B;
        last = B;
    }
    memcpy(m->logits, m->logits_b + (size_t)(last - 1) * V, (size_t)V * sizeof(float));
    dump(dir, "prefill_logits.f32", m->logits, (size_t)V * sizeof(float));
    uint32_t *out = calloc(n_gen, 4);
    float *gap = calloc(n_gen, 4);
    for (uint32_t i = 0; i < n_gen; i++) {
        out[i] = top2(m->logits, V, &gap[i]);
        fprintf(stderr, "[greedy] %u: token %u gap %.4f\n", i, out[i], gap[i]);
        if (i + 1 < n_gen) model_forward(m, pool, out[i], n_prompt + i);
    }
    dump(dir, "stream.u32", out, (size_t)n_gen * 4);
    dump(dir, "gap.f32", gap, (size_t)n_gen * 4);
    pool_destroy(pool);
    model_free(m);
    free(m); free(out); free(gap);
    return 0;
}

/* the spec loop of main.c:166-225 (k <= SPEC_MAX_B-1) */
static uint32_t spec_batch(qwen_model_t *m, uint32_t k, uint32_t n_ctx, uint32_t n_predict,
                           uint32_t *out, uint32_t *js, uint32_t *ncyc)
{
    const uint32_t V = m->cfg.vocab_size;
    const float *last = m->logits;
    uint32_t gen = 0, cyc = 0;
    while (gen < n_predict) {
        const uint32_t P = m->pos - 1, room = n_ctx - 1 - P;
        if (room < 1) break;
        const uint32_t kk = k < room - 1 ? k : room - 1;
        uint32_t cand[SPEC_MAX_B];
        cand[0] = model_sample_greedy(last, V);
        for (uint32_t s = 1; s <= kk; s++) {
            mtp_forward(m, g_pool, cand[s - 1], P + s, 1);
            cand[s] = model_sample_greedy(m->logits, V);
        }
        model_forward_batch(m, g_pool, cand, P + 1, kk + 1, 1);
        uint32_t j = kk;
        for (uint32_t i = 0; i < kk; i++)
            if (model_sample_greedy(m->logits_b + (size_t)i * V, V) != cand[i + 1]) { j = i; break; }
        for (uint32_t i = 0; i <= j && gen < n_predict; i++) out[gen++] = cand[i];
        js[cyc] = j;
        if (m->pos >= n_ctx) { cyc++; break; }
        if (j < kk) { model_rollback_to(m, j); m->pos = P + j + 2; }
        memcpy(m->mtp_h, m->h_save + (size_t)j * m->dims.n_embd, m->dims.n_embd * sizeof(float));
        mtp_forward(m, g_pool, cand[j], P + j + 1, 0);
        last = m->logits_b + (size_t)j * V;
        cyc++;
    }
    *ncyc = cyc;
    return gen;
}

/* Same stream for any k: drafts as main.c:182-185, verification by single-token
 * forwards that stop at the first mismatch (no rollback needed), MTP anchored on
 * the backbone hidden state after the last accepted token (debug_spec.c:26).
 * The context-end test is main.c's: after a batched verify of kk+1 tokens the
 * position is P+kk+2, and the loop stops once that reaches n_ctx (main.c:210).
 * force (no reference counterpart; the device loop's benchmark modes): 1 = every
 * draft accepted (j = kk), 2 = j = cycle mod (kk+1); verification then forwards
 * cand[0..j] whatever the backbone predicts.  last/mtph (optional) receive the
 * logits the next cycle would start from and the MTP hidden state at the end. */
static uint32_t spec_seq(qwen_model_t *m, uint32_t k, uint32_t n_ctx, uint32_t n_predict, int force,
                         uint32_t *out, uint32_t *js, uint32_t *ncyc, float *last_out, float *mtph_out)
{
    const uint32_t V = m->cfg.vocab_size, E = m->dims.n_embd;
    float *last = malloc(V * sizeof(float)), *h = malloc(E * sizeof(float));
    memcpy(last, m->logits, V * sizeof(float));
    uint32_t gen = 0, cyc = 0, cand[16];
    while (gen < n_predict) {
        const uint32_t P = m->pos - 1, room = n_ctx - 1 - P;
        if (room < 1) break;
        const uint32_t kk = k < room - 1 ? k : room - 1;
        cand[0] = model_sample_greedy(last, V);
        for (uint32_t s = 1; s <= kk; s++) {
            mtp_forward(m, g_pool, cand[s - 1], P + s, 1);
            cand[s] = model_sample_greedy(m->logits, V);
        }
        const uint32_t jf = force == 1 ? kk : force == 2 ? cyc % (kk + 1) : kk;
        uint32_t j = jf;
        for (uint32_t i = 0; i <= jf; i++) {
            model_forward(m, g_pool, cand[i], P + 1 + i);
            memcpy(last, m->logits, V * sizeof(float));
            memcpy(h, m->x, E * sizeof(float));
            if (!force && i < kk && model_sample_greedy(last, V) != cand[i + 1]) { j = i; break; }
        }
        for (uint32_t i = 0; i <= j && gen < n_predict; i++) out[gen++] = cand[i];
        js[cyc] = j;
        if (P + kk + 2 >= n_ctx) { cyc++; break; }
        memcpy(m->mtp_h, h, E * sizeof(float));
        mtp_forward(m, g_pool, cand[j], P + j + 1, 0);
        cyc++;
    }
    if (last_out) memcpy(last_out, last, V * sizeof(float));
    if (mtph_out) memcpy(mtph_out, m->mtp_h, E * sizeof(float));
    free(last); free(h);
    *ncyc = cyc;
    return gen;
}

/* spec mode: every speculative scenario on one model, prompt of n_prompt ids.
 * long_form (an n_ctx-sized prompt): the prefill's last logits, then natural
 * and all-accepted streams for k = 1, 3, 5, 7 only, with sequential verification. */
static int spec_mode(const char *path, const char *dir, uint32_t n_ctx, uint32_t n_prompt, uint32_t n_predict,
                     int long_form)
{
    qwen_model_t *m = calloc(1, sizeof *m);
    if (!m || model_init(m, path, n_ctx)) return 1;
    if (long_form) {
        const long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
        g_pool = pool_create(ncpu > 0 ? (int)ncpu : 1, 1);
    }
    const uint32_t V = m->cfg.vocab_size, E = m->dims.n_embd;
    uint32_t *prompt = malloc((size_t)n_prompt * 4), *out = calloc(n_predict + 16, 4), *js = calloc(n_predict + 16, 4);
    uint32_t nc, ng;
    float *last = malloc((size_t)V * 4), *mtph = malloc((size_t)E * 4);
    for (uint32_t i = 0; i < n_prompt; i++) prompt[i] = prompt_tok(i, V);
    dump(dir, "prompt.u32", prompt, n_prompt * 4);
    char name[96];
#define DUMP4(FMT, ...) do { snprintf(name, sizeof name, FMT ".u32", __VA_ARGS__); dump(dir, name, out, ng * 4); \
        snprintf(name, sizeof name, FMT "_j.u32", __VA_ARGS__); dump(dir, name, js, nc * 4); \
        snprintf(name, sizeof name, FMT "_last.f32", __VA_ARGS__); dump(dir, name, last, (size_t)V * 4); \
        snprintf(name, sizeof name, FMT "_mtph.f32", __VA_ARGS__); dump(dir, name, mtph, (size_t)E * 4); } while (0)
    if (long_form) {
        prefill(m, prompt, n_prompt, 1);
        dump(dir, "prefill_last.f32", m->logits, (size_t)V * 4);
    }
    for (uint32_t k = 1; k <= 2 && !long_form; k++) {               /* main.c's own loop */
        model_free(m);
        if (model_init(m, path, n_ctx)) return 1;
        prefill(m, prompt, n_prompt, 1);
        ng = spec_batch(m, k, n_ctx, n_predict, out, js, &nc);
        memcpy(last, m->logits_b + (size_t)js[nc - 1] * V, (size_t)V * 4);
        memcpy(mtph, m->mtp_h, (size_t)E * 4);
        DUMP4("spec_k%u", k);
    }
    for (int force = 0; force <= 2; force++)
        for (uint32_t k = 1; k <= 7; k++) {
            if (long_form && (force == 2 || !(k & 1))) continue;
            model_free(m);
            if (model_init(m, path, n_ctx)) return 1;
            prefill(m, prompt, n_prompt, 1);
            ng = spec_seq(m, k, n_ctx, n_predict, force, out, js, &nc, last, mtph);
            if (force) DUMP4("spec_f%d_k%u", force, k);
            else DUMP4("spec_seq_k%u", k);
        }
#undef DUMP4
    model_free(m);
    if (model_init(m, path, n_ctx)) return 1;          /* plain greedy stream, k tokens past n_predict */
    prefill(m, prompt, n_prompt, 0);
    uint32_t cur = model_sample_greedy(m->logits, V);
    ng = 0;
    out[ng++] = cur;
    while (ng < n_predict + 8 && m->pos < n_ctx) {
        model_forward(m, g_pool, cur, m->pos);
        cur = model_sample_greedy(m->logits, V);
        out[ng++] = cur;
    }
    dump(dir, "greedy.u32", out, ng * 4);
    model_free(m);
    free(m); free(prompt); free(out); free(js); free(last); free(mtph);
    return 0;
}

int main(int argc, char **argv)
{
    if (argc < 4) { fprintf(stderr, "usage: %s model.gguf outdir n_ctx\n", argv[0]); return 1; }
    if (argc >= 7 && !strcmp(argv[4], "greedy")) return greedy_mode(argv[1], argv[2], (uint32_t)atoi(argv[3]), argv[5],
                                                                  (uint32_t)atoi(argv[6]));
    if (argc >= 7 && (!strcmp(argv[4], "spec") || !strcmp(argv[4], "long")))
        return spec_mode(argv[1], argv[2], (uint32_t)atoi(argv[3]), (uint32_t)atoi(argv[5]), (uint32_t)atoi(argv[6]),
                         !strcmp(argv[4], "long"));
    const char *path = argv[1], *dir = argv[2];
    const uint32_t n_ctx = (uint32_t)atoi(argv[3]);
    qwen_model_t *m = calloc(1, sizeof *m);
    if (model_init(m, path, n_ctx)) return 1;
    const uint32_t V = m->cfg.vocab_size, E = m->dims.n_embd;
    uint32_t prompt[64];
    for (uint32_t i = 0; i < 64; i++) prompt[i] = prompt_tok(i, V);
    dump(dir, "prompt.u32", prompt, sizeof prompt);

    /* sequential vs batched forward of prompt[0..7] */
    float *seq = malloc((size_t)8 * V * sizeof(float));
    for (uint32_t i = 0; i < 8; i++) {
        model_forward(m, g_pool, prompt[i], i);
        memcpy(seq + (size_t)i * V, m->logits, V * sizeof(float));
    }
    dump(dir, "seq_logits.f32", seq, (size_t)8 * V * sizeof(float));
    model_free(m);
    if (model_init(m, path, n_ctx)) return 1;
    model_forward_batch(m, g_pool, prompt, 0, 8, 0);
    dump(dir, "batch_logits.f32", m->logits_b, (size_t)8 * V * sizeof(float));
    dump(dir, "batch_hsave.f32", m->h_save, (size_t)8 * E * sizeof(float));
    /* MTP: prefill the MTP KV for prompt[0..7] then one draft with logits */
    mtp_forward_batch(m, g_pool, prompt, 0, 8, 0);
    mtp_forward(m, g_pool, prompt[8], 8, 1);
    dump(dir, "mtp_logits.f32", m->logits, V * sizeof(float));
    dump(dir, "mtp_h.f32", m->mtp_h, E * sizeof(float));
    model_free(m);

    /* rollback (debug_rollback.c:25-57 pattern) on prompt[0..4] */
    if (model_init(m, path, n_ctx)) return 1;
    for (uint32_t i = 0; i < 5; i++) model_forward(m, g_pool, prompt[i], i);
    uint32_t c1[3] = { prompt[10], prompt[11], prompt[12] }, c2[3] = { prompt[13], prompt[14], prompt[15] };
    model_forward_batch(m, g_pool, c1, 5, 3, 1);
    model_rollback_to(m, 1);
    m->pos = 5 + 1 + 2;
    model_forward_batch(m, g_pool, c2, 7, 3, 1);
    dump(dir, "rollback_logits.f32", m->logits_b, (size_t)3 * V * sizeof(float));
    model_free(m);

    const uint32_t n_prompt = 20, n_predict = 40;
    uint32_t out[256], js[256], nc, ng;
    char name[64];
    for (uint32_t k = 1; k <= 2; k++) {
        if (model_init(m, path, n_ctx)) return 1;
        prefill(m, prompt, n_prompt, 1);
        memset(out, 0, sizeof out); memset(js, 0, sizeof js);
        ng = spec_batch(m, k, n_ctx, n_predict, out, js, &nc);
        snprintf(name, sizeof name, "spec_k%u.u32", k); dump(dir, name, out, ng * 4);
        snprintf(name, sizeof name, "spec_j_k%u.u32", k); dump(dir, name, js, nc * 4);
        model_free(m);
    }
    for (uint32_t k = 1; k <= 7; k++) {
        if (model_init(m, path, n_ctx)) return 1;
        prefill(m, prompt, n_prompt, 1);
        memset(out, 0, sizeof out); memset(js, 0, sizeof js);
        ng = spec_seq(m, k, n_ctx, n_predict, 0, out, js, &nc, NULL, NULL);
        snprintf(name, sizeof name, "spec_seq_k%u.u32", k); dump(dir, name, out, ng * 4);
        snprintf(name, sizeof name, "spec_seq_j_k%u.u32", k); dump(dir, name, js, nc * 4);
        model_free(m);
    }
    /* plain greedy stream */
    if (model_init(m, path, n_ctx)) return 1;
    prefill(m, prompt, n_prompt, 0);
    uint32_t cur = model_sample_greedy(m->logits, V);
    out[0] = cur;
    for (uint32_t i = 1; i < n_predict; i++) {
        model_forward(m, g_pool, cur, m->pos);
        cur = model_sample_greedy(m->logits, V);
        out[i] = cur;
    }
    dump(dir, "greedy.u32", out, n_predict * 4);
    model_free(m);
    /* sampled streams: temp, top_p, top_k, repeat_penalty, seed (main.c:108, 232-248) */
    static const struct { float temp, top_p; uint32_t top_k; float pen; uint64_t seed; } SAMPLE_CFG[4] = {
        { 0.8f, 0.9f, 40, 1.1f, 7 }, { 1.0f, 1.0f, 0, 1.0f, 99 }, { 0.5f, 0.5f, 5, 1.3f, 12345 },
        { 1.2f, 0.95f, 300, 1.05f, 42 } };
    double cfg[4][5];
    for (uint32_t c = 0; c < 4; c++) {
        cfg[c][0] = SAMPLE_CFG[c].temp; cfg[c][1] = SAMPLE_CFG[c].top_p; cfg[c][2] = SAMPLE_CFG[c].top_k;
        cfg[c][3] = SAMPLE_CFG[c].pen; cfg[c][4] = (double)SAMPLE_CFG[c].seed;
    }
    dump(dir, "sample_cfg.f64", cfg, sizeof cfg);
    for (uint32_t c = 0; c < 4; c++) {
        if (model_init(m, path, n_ctx)) return 1;
        prefill(m, prompt, n_prompt, 0);
        sampler_t *smp = sampler_init(SAMPLE_CFG[c].temp, SAMPLE_CFG[c].top_p, SAMPLE_CFG[c].top_k, SAMPLE_CFG[c].pen,
                                      SAMPLE_CFG[c].seed);
        uint32_t all[256];
        memcpy(all, prompt, n_prompt * sizeof(uint32_t));
        size_t n_all = n_prompt;
        uint32_t gen = 0;
        cur = sampler_sample(smp, m->logits, V, all, n_all);
        all[n_all++] = cur;
        out[gen++] = cur;
        for (uint32_t i = 1; i < n_predict; i++) {
            if (m->pos >= n_ctx) break;
            model_forward(m, g_pool, cur, m->pos);
            cur = sampler_sample(smp, m->logits, V, all, n_all);
            all[n_all++] = cur;
            out[gen++] = cur;
        }
        snprintf(name, sizeof name, "sample_c%u.u32", c);
        dump(dir, name, out, gen * 4);
        sampler_free(smp);
        model_free(m);
    }
    free(m); free(seq);
    return 0;
}
