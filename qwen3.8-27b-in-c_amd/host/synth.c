/*
 * synth.c -- deterministic random-init model weights and GGUF writer
 * (include/qwen_synth.h).  Tensor names, shapes and metadata keys are the ones
 * the reference loader binds (reference model.c:85-143,245-274, gguf.c:91-110)
 * so a file written here loads unmodified in both engines.
 */
#define _POSIX_C_SOURCE 200809L
#include "qwen_synth.h"
#include "quant.h"
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ RNG */
static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline uint64_t stream_base(uint64_t seed, uint64_t id)
{
    return mix64(seed ^ mix64(id * 0xD1B54A32D192ED03ull + 0x8CB92BA72F3D8DD7ull));
}
static inline uint64_t block_key(uint64_t base, uint64_t blk)
{
    return mix64(base + (blk + 1) * 0x9E3779B97F4A7C15ull);
}
static inline uint64_t word(uint64_t key, uint32_t i)
{
    return mix64(key ^ ((uint64_t)(i + 1) * 0xA0761D6478BD642Full));
}
/* Irwin-Hall(12) standard normal from words w, w+1, w+2 of the block stream:
 * z = (sum of twelve 16-bit uniforms - 393210) / 65536, exact in float. */
static inline float normal3(uint64_t key, uint32_t w)
{
    int32_t s = 0;
    for (uint32_t k = 0; k < 3; k++) {
        const uint64_t v = word(key, w + k);
        s += (int32_t)(v & 0xFFFF) + (int32_t)((v >> 16) & 0xFFFF) +
             (int32_t)((v >> 32) & 0xFFFF) + (int32_t)(v >> 48);
    }
    return (float)(s - 393210) * (1.0f / 65536.0f);
}

uint16_t qwen_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u)                                   /* inf / nan */
        return sign | 0x7C00u | (ax > 0x7F800000u ? (uint16_t)(0x200u | ((ax >> 13) & 0x3FFu)) : 0);
    if (ax >= 0x477FF000u) return sign | 0x7C00u;            /* rounds past 65504 */
    if (ax >= 0x38800000u)                                   /* normal half */
        return sign | (uint16_t)((ax - 0x38000000u + 0xFFFu + ((ax >> 13) & 1u)) >> 13);
    const uint32_t e = ax >> 23;                             /* subnormal half or zero */
    if (e < 102) return sign;
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u, s = 126 - e;
    uint32_t r = m >> s;
    const uint32_t rem = m & ((1u << s) - 1u), half = 1u << (s - 1);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return sign | (uint16_t)r;
}

static inline void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline void put_words(uint8_t *p, uint64_t key, uint32_t w0, size_t n)
{
    for (size_t i = 0; i < n; i += 8) {
        const uint64_t v = word(key, w0 + (uint32_t)(i / 8));
        const size_t k = n - i < 8 ? n - i : 8;
        memcpy(p + i, &v, k);
    }
}

/* one quantised block from its key; sd = sigma of the super-block scale d */
static void gen_block(int32_t type, uint64_t key, float sd, uint8_t *b)
{
    switch (type) {
    case GGML_IQ4_XS:                   /* d | scales_h | scales_l[4] | qs[128] */
        put16(b, qwen_f32_to_f16(fabsf(normal3(key, 0)) * sd));
        put_words(b + 2, key, 3, 6);
        put_words(b + 8, key, 4, 128);
        break;
    case GGML_Q4_K:                     /* d | dmin | scales[12] | qs[128] */
        put16(b, qwen_f32_to_f16(fabsf(normal3(key, 0)) * sd));
        put16(b + 2, qwen_f32_to_f16(fabsf(normal3(key, 3)) * sd * 4.0f));
        put_words(b + 4, key, 6, 12);
        put_words(b + 16, key, 8, 128);
        break;
    case GGML_Q5_K:                     /* d | dmin | scales[12] | qh[32] | qs[128] */
        put16(b, qwen_f32_to_f16(fabsf(normal3(key, 0)) * sd));
        put16(b + 2, qwen_f32_to_f16(fabsf(normal3(key, 3)) * sd * 4.0f));
        put_words(b + 4, key, 6, 12);
        put_words(b + 16, key, 8, 32);
        put_words(b + 48, key, 12, 128);
        break;
    case GGML_Q6_K:                     /* ql[128] | qh[64] | scales[16] | d */
        put_words(b, key, 3, 208);
        put16(b + 208, qwen_f32_to_f16(fabsf(normal3(key, 0)) * sd));
        break;
    case GGML_Q8_0:                     /* d | qs[32] */
        put16(b, qwen_f32_to_f16(fabsf(normal3(key, 0)) * sd));
        put_words(b + 2, key, 3, 32);
        break;
    default:
        break;
    }
}

static uint64_t elems_per_block(int32_t t)
{
    return t == GGML_Q8_0 ? 32 : (t == GGML_F32 ? 1 : 256);
}

typedef struct {
    int32_t type; uint64_t nblk, b0, b1, base; float sd; uint8_t *out; size_t bs;
} fill_job;

static void *fill_worker(void *p)
{
    fill_job *j = p;
    for (uint64_t b = j->b0; b < j->b1; b++) {
        if (j->type == GGML_F32) {
            const float v = normal3(block_key(j->base, b), 0) * j->sd;
            memcpy(j->out + b * 4, &v, 4);
        } else {
            gen_block(j->type, block_key(j->base, b), j->sd, j->out + b * j->bs);
        }
    }
    return NULL;
}

int qwen_synth_matrix(int32_t type, uint64_t ne0, uint64_t ne1, uint64_t seed, uint64_t id,
                      float sigma_d, void *out, int n_threads)
{
    const size_t bs = quant_block_size((ggml_type_t)type);
    const uint64_t epb = elems_per_block(type);
    if (!bs || ne0 % epb) return -1;
    const uint64_t nblk = ne0 / epb * ne1;
    if (n_threads <= 0) {
        long c = sysconf(_SC_NPROCESSORS_ONLN);
        n_threads = c > 16 ? 16 : (c < 1 ? 1 : (int)c);
    }
    if (nblk < 4096) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    fill_job jobs[64];
    const uint64_t base = stream_base(seed, id);
    for (int k = 0; k < n_threads; k++) {
        jobs[k] = (fill_job){ type, nblk, nblk * (uint64_t)k / (uint64_t)n_threads,
                              nblk * (uint64_t)(k + 1) / (uint64_t)n_threads, base, sigma_d,
                              (uint8_t *)out, bs };
        if (n_threads == 1) fill_worker(&jobs[k]);
        else pthread_create(&th[k], NULL, fill_worker, &jobs[k]);
    }
    if (n_threads > 1)
        for (int k = 0; k < n_threads; k++) pthread_join(th[k], NULL);
    return 0;
}

void qwen_synth_normal(float *out, uint64_t n, uint64_t seed, uint64_t id, float mu, float sigma)
{
    const uint64_t base = stream_base(seed, id);
    for (uint64_t i = 0; i < n; i++) out[i] = mu + sigma * normal3(block_key(base, i), 0);
}

/* ------------------------------------------------------------ model spec */
void qwen_synth_spec_27b(qwen_synth_spec_t *s, uint64_t seed)
{
    memset(s, 0, sizeof *s);
    s->n_embd = 5120; s->n_ff = 17408; s->n_layer = 64;
    s->n_head = 24; s->n_kv_head = 4; s->head_dim = 256;
    s->n_k_heads = 16; s->n_v_heads = 48; s->state = 128;
    s->vocab = 248320; s->rope_dim = 64; s->full_attn_interval = 4; s->context_len = 262144;
    s->rope_theta = 10000000.0f; s->eps = 1e-6f;
    s->type_default = GGML_IQ4_XS;
    s->type_embd = s->type_output = s->type_qkv = s->type_eh_proj = -1;
    s->gain_output = 4.0f;
    s->seed = seed;
}

void qwen_synth_spec_tiny(qwen_synth_spec_t *s, uint64_t seed, int variant)
{
    const int mixed = variant == 1;
    memset(s, 0, sizeof *s);
    s->n_embd = 256; s->n_ff = 2048; s->n_layer = 8;   /* n_ff >= max(conv_dim, 2*n_head*head_dim, 2*n_embd): the reference batch arenas use stride n_ff (model.c:207) */
    s->n_head = 4; s->n_kv_head = 2; s->head_dim = 256;
    s->n_k_heads = 2; s->n_v_heads = 4; s->state = 128;
    s->vocab = 1024; s->rope_dim = 64; s->full_attn_interval = 4; s->context_len = 4096;
    s->rope_theta = 10000000.0f; s->eps = 1e-6f;
    s->type_default = GGML_IQ4_XS;
    s->type_embd = s->type_output = s->type_qkv = s->type_eh_proj = -1;
    if (mixed) {                         /* the real checkpoint's format mix */
        s->type_embd = GGML_Q4_K; s->type_output = GGML_Q6_K;
        s->type_qkv = GGML_Q5_K; s->type_eh_proj = GGML_Q8_0;
    }
    s->gain_output = 4.0f;
    s->seed = seed;
    if (variant == 2) {                  /* drafts that the backbone mostly accepts */
        s->gain_embd = 5.0f;
        s->mtp_diag = 1;
        s->tie_shift = 1;
    }
}

/* RMS of one decoded weight per unit d, per format (uniform random codes):
 * used to pick sigma_d so a unit-RMS input gives a ~unit-RMS output. */
static float code_rms(int32_t t)
{
    switch (t) {
    case GGML_IQ4_XS: return 67.44f * 18.48f;    /* rms(codebook) * rms(ls-32) */
    case GGML_Q4_K: return 36.5f * 8.80f;
    case GGML_Q5_K: return 36.5f * 18.0f;
    case GGML_Q6_K: return 73.9f * 18.5f;
    case GGML_Q8_0: return 73.9f;
    default: return 1.0f;
    }
}

enum { K_MAT, K_NORM, K_CONV, K_DTB, K_SSMA };

typedef struct { char name[GGUF_MAX_NAME]; uint32_t nd; uint64_t ne0, ne1; int32_t type; int kind; float gain; } tdesc;

static int32_t pick(int32_t over, int32_t dflt) { return over >= 0 ? over : dflt; }

/* canonical tensor order; returns count, fills d[i] when d != NULL */
static uint32_t enumerate(const qwen_synth_spec_t *s, tdesc *d)
{
    uint32_t n = 0;
    const uint64_t E = s->n_embd, F = s->n_ff, V = s->vocab;
    const uint64_t di = (uint64_t)s->n_v_heads * s->state;
    const uint64_t cd = 2ull * s->n_k_heads * s->state + di;
    const int32_t T = s->type_default;
#define ADD(NAME_FMT, IDX, ND, A, B, TY, KIND, GAIN) do { \
        if (d) { snprintf(d[n].name, GGUF_MAX_NAME, NAME_FMT, IDX); d[n].nd = ND; d[n].ne0 = A; \
                 d[n].ne1 = B; d[n].type = TY; d[n].kind = KIND; d[n].gain = GAIN; } n++; } while (0)
    const float ge = s->gain_embd > 0.0f ? s->gain_embd : 1.0f;
    const float gr = s->gain_resid > 0.0f ? s->gain_resid : 0.5f;
    ADD("token_embd.weight%.0u", 0u, 2, E, V, pick(s->type_embd, T), K_MAT, ge);
    ADD("output_norm.weight%.0u", 0u, 1, E, 1, GGML_F32, K_NORM, 1.0f);
    if (!s->tie_output) ADD("output.weight%.0u", 0u, 2, E, V, pick(s->type_output, T), K_MAT, s->gain_output);
    for (uint32_t il = 0; il <= s->n_layer; il++) {
        const int mtp = il == s->n_layer;
        const int rec = !mtp && ((il + 1) % s->full_attn_interval) != 0;
        ADD("blk.%u.attn_norm.weight", il, 1, E, 1, GGML_F32, K_NORM, 1.0f);
        ADD("blk.%u.post_attention_norm.weight", il, 1, E, 1, GGML_F32, K_NORM, 1.0f);
        ADD("blk.%u.ffn_gate.weight", il, 2, E, F, T, K_MAT, 1.0f);
        ADD("blk.%u.ffn_up.weight", il, 2, E, F, T, K_MAT, 1.0f);
        ADD("blk.%u.ffn_down.weight", il, 2, F, E, T, K_MAT, gr);
        if (rec) {
            ADD("blk.%u.attn_qkv.weight", il, 2, E, cd, pick(s->type_qkv, T), K_MAT, 1.0f);
            ADD("blk.%u.attn_gate.weight", il, 2, E, di, T, K_MAT, 1.0f);
            ADD("blk.%u.ssm_conv1d.weight", il, 2, 4, cd, GGML_F32, K_CONV, 1.0f);
            ADD("blk.%u.ssm_dt.bias", il, 1, s->n_v_heads, 1, GGML_F32, K_DTB, 1.0f);
            ADD("blk.%u.ssm_a", il, 1, s->n_v_heads, 1, GGML_F32, K_SSMA, 1.0f);
            ADD("blk.%u.ssm_beta.weight", il, 2, E, s->n_v_heads, T, K_MAT, 1.0f);
            ADD("blk.%u.ssm_alpha.weight", il, 2, E, s->n_v_heads, T, K_MAT, 1.0f);
            ADD("blk.%u.ssm_norm.weight", il, 1, s->state, 1, GGML_F32, K_NORM, 1.0f);
            ADD("blk.%u.ssm_out.weight", il, 2, di, E, T, K_MAT, gr);
        } else {
            ADD("blk.%u.attn_q.weight", il, 2, E, 2ull * s->n_head * s->head_dim, T, K_MAT, 1.0f);
            ADD("blk.%u.attn_k.weight", il, 2, E, (uint64_t)s->n_kv_head * s->head_dim, T, K_MAT, 1.0f);
            ADD("blk.%u.attn_v.weight", il, 2, E, (uint64_t)s->n_kv_head * s->head_dim, T, K_MAT, 1.0f);
            ADD("blk.%u.attn_q_norm.weight", il, 1, s->head_dim, 1, GGML_F32, K_NORM, 1.0f);
            ADD("blk.%u.attn_k_norm.weight", il, 1, s->head_dim, 1, GGML_F32, K_NORM, 1.0f);
            ADD("blk.%u.attn_output.weight", il, 2, (uint64_t)s->n_head * s->head_dim, E, T, K_MAT, gr);
        }
        if (mtp) {
            ADD("blk.%u.nextn.eh_proj.weight", il, 2, 2 * E, E, pick(s->type_eh_proj, T), K_MAT, 1.0f);
            ADD("blk.%u.nextn.enorm.weight", il, 1, E, 1, GGML_F32, K_NORM, 1.0f);
            ADD("blk.%u.nextn.hnorm.weight", il, 1, E, 1, GGML_F32, K_NORM, 1.0f);
            ADD("blk.%u.nextn.shared_head_norm.weight", il, 1, E, 1, GGML_F32, K_NORM, 1.0f);
        }
    }
    /* a copy of token_embd (same type and bytes) as the last tensor */
    if (s->tie_output == 2) ADD("output.weight%.0u", 0u, 2, E, V, pick(s->type_embd, T), K_MAT, ge);
#undef ADD
    return n;
}

uint32_t qwen_synth_count(const qwen_synth_spec_t *s) { return enumerate(s, NULL); }

int qwen_synth_describe(const qwen_synth_spec_t *s, uint32_t i, qwen_synth_tensor_t *o)
{
    const uint32_t n = enumerate(s, NULL);
    if (i >= n) return -1;
    tdesc *d = calloc(n, sizeof *d);
    enumerate(s, d);
    memset(o, 0, sizeof *o);
    memcpy(o->name, d[i].name, GGUF_MAX_NAME);
    o->n_dims = d[i].nd;
    o->ne[0] = d[i].ne0;
    o->ne[1] = d[i].ne1;
    o->type = d[i].type;
    o->nbytes = quant_row_bytes((ggml_type_t)d[i].type, d[i].ne0) * d[i].ne1;
    switch (d[i].kind) {
    case K_NORM: o->mu = 1.0f; o->sigma = s->norm_sigma > 0.0f ? s->norm_sigma : 0.1f; break;
    case K_CONV: o->mu = 0.0f; o->sigma = 0.5f; break;
    case K_DTB:  o->mu = 0.0f; o->sigma = 0.5f; break;
    case K_SSMA: o->mu = 0.5f; o->sigma = 0.5f; o->neg_abs = 1; break;
    default:     o->mu = 0.0f;
                 o->sigma = d[i].gain / (code_rms(d[i].type) * sqrtf((float)d[i].ne0)); break;
    }
    free(d);
    return 0;
}

/* IQ4_XS eh_proj [2E -> E] whose token half is ~identity: in row r every
 * 32-element sub-block of the first E columns has scale code 32 (weights 0)
 * except the one holding column r, code 63, with nibble 15 (codebook 113) at
 * column r and nibble 8 (codebook 1) elsewhere; d = 1/(31*113), so W[r][r] ~ 1
 * and its 31 neighbours ~ 0.009.  The hidden half keeps the random codes with
 * scale codes drawn from 31..33 and d/8, i.e. weights of at most 127 d/8 ~ 0.0045. */
static int diag_eh_proj(const qwen_synth_tensor_t *t, uint64_t seed, uint32_t id, uint8_t *out)
{
    if (t->type != GGML_IQ4_XS || t->ne[0] % 512 || t->ne[1] * 2 != t->ne[0]) return -1;
    const uint64_t E = t->ne[1], nsb = t->ne[0] / 256;
    const uint64_t base = stream_base(seed, (uint64_t)id ^ 0x5EEDull);
    const uint16_t d = qwen_f32_to_f16(1.0f / (31.0f * 113.0f)), dh = qwen_f32_to_f16(1.0f / (8.0f * 31.0f * 113.0f));
    for (uint64_t r = 0; r < E; r++)
        for (uint64_t sb = 0; sb < nsb; sb++) {
            uint8_t *b = out + (r * nsb + sb) * 136;
            uint16_t sh = 0;
            uint8_t sl[4] = { 0, 0, 0, 0 };
            if (sb * 256 < E) {                       /* token half */
                const int hit = r / 256 == sb;
                const uint32_t ib_r = (uint32_t)(r % 256) / 32, jj = (uint32_t)(r % 32);
                for (uint32_t ib = 0; ib < 8; ib++) {
                    const uint32_t ls = (hit && ib == ib_r) ? 63u : 32u;
                    sl[ib / 2] |= (uint8_t)((ls & 15u) << (4 * (ib % 2)));
                    sh |= (uint16_t)(((ls >> 4) & 3u) << (2 * ib));
                }
                memset(b + 8, 0x88, 128);
                if (hit) {
                    uint8_t *q = b + 8 + 16 * ib_r + (jj % 16);
                    *q = jj < 16 ? (uint8_t)((*q & 0xF0) | 0x0F) : (uint8_t)((*q & 0x0F) | 0xF0);
                }
                put16(b, d);
            } else {                                  /* hidden half: weak random */
                const uint64_t key = block_key(base, r * nsb + sb);
                for (uint32_t ib = 0; ib < 8; ib++) {
                    const uint32_t ls = 31u + (uint32_t)(word(key, 40 + ib) % 3u);
                    sl[ib / 2] |= (uint8_t)((ls & 15u) << (4 * (ib % 2)));
                    sh |= (uint16_t)(((ls >> 4) & 3u) << (2 * ib));
                }
                put_words(b + 8, key, 4, 128);
                put16(b, dh);
            }
            put16(b + 2, sh);
            memcpy(b + 4, sl, 4);
        }
    return 0;
}

/* token_embd of a tie_shift model (IQ4_XS): random codes with one super-block
 * scale d for every block, so all rows have about the same norm and no output
 * row outweighs the others for every input */
static int tied_embd(const qwen_synth_spec_t *s, void *out)
{
    qwen_synth_tensor_t e;
    if (qwen_synth_describe(s, 0, &e) || e.type != GGML_IQ4_XS) return -1;
    if (qwen_synth_matrix(e.type, e.ne[0], e.ne[1], s->seed, 0, e.sigma, out, 0)) return -1;
    const uint16_t d = qwen_f32_to_f16(e.sigma);
    for (uint64_t b = 0; b < e.nbytes / 136; b++) put16((uint8_t *)out + b * 136, d);
    return 0;
}

int qwen_synth_fill(const qwen_synth_spec_t *s, uint32_t i, void *out)
{
    qwen_synth_tensor_t t;
    if (qwen_synth_describe(s, i, &t)) return -1;
    if (s->mtp_diag && strstr(t.name, ".nextn.eh_proj.weight"))
        return diag_eh_proj(&t, s->seed, i, out);
    if (s->tie_shift && i == 0) return tied_embd(s, out);
    if (s->tie_output == 2 && !strcmp(t.name, "output.weight")) return qwen_synth_fill(s, 0, out);
    if (s->tie_shift && !strcmp(t.name, "output.weight")) {
        qwen_synth_tensor_t e;                    /* token_embd is tensor 0 */
        if (qwen_synth_describe(s, 0, &e) || e.type != t.type || e.nbytes != t.nbytes || e.ne[1] < 2) return -1;
        uint8_t *emb = malloc(e.nbytes);
        if (!emb || tied_embd(s, emb)) { free(emb); return -1; }
        const size_t rb = e.nbytes / e.ne[1];
        memcpy(out, emb + (e.ne[1] - 1) * rb, rb);
        memcpy((uint8_t *)out + rb, emb, (e.ne[1] - 1) * rb);
        free(emb);
        return 0;
    }
    if (t.type != GGML_F32)
        return qwen_synth_matrix(t.type, t.ne[0], t.ne[1], s->seed, i, t.sigma, out, 0);
    const uint64_t n = t.ne[0] * t.ne[1];
    float *f = out;
    qwen_synth_normal(f, n, s->seed, i, 0.0f, 1.0f);
    for (uint64_t k = 0; k < n; k++)
        f[k] = t.neg_abs ? -(t.mu + t.sigma * fabsf(f[k])) : t.mu + t.sigma * f[k];
    return 0;
}

/* ------------------------------------------------------------ GGUF writer */
static int w_bytes(FILE *f, const void *p, size_t n) { return fwrite(p, 1, n, f) == n ? 0 : -1; }
static int w_u32(FILE *f, uint32_t v) { return w_bytes(f, &v, 4); }
static int w_u64(FILE *f, uint64_t v) { return w_bytes(f, &v, 8); }
static int w_str(FILE *f, const char *s) { uint64_t n = strlen(s); return w_u64(f, n) || w_bytes(f, s, n); }
static int kv_u32(FILE *f, const char *k, uint32_t v) { return w_str(f, k) || w_u32(f, GGUF_TYPE_UINT32) || w_u32(f, v); }
static int kv_f32(FILE *f, const char *k, float v) { return w_str(f, k) || w_u32(f, GGUF_TYPE_FLOAT32) || w_bytes(f, &v, 4); }

/* The byte-level symbol of byte b (the GPT-2 byte-to-unicode map): the printable
 * bytes '!'..'~', 0xA1..0xAC and 0xAE..0xFF stand for themselves, every other
 * byte for code point 256 + its rank among those others; as UTF-8 in out[4]. */
static void byte_symbol(int b, char out[4])
{
    int cp = b, rank = 0;
    const int printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
    if (!printable) {
        for (int c = 0; c < b; c++)
            if (!((c >= '!' && c <= '~') || (c >= 0xA1 && c <= 0xAC) || (c >= 0xAE && c <= 0xFF))) rank++;
        cp = 256 + rank;
    }
    if (cp < 0x80) { out[0] = (char)cp; out[1] = 0; }
    else { out[0] = (char)(0xC0 | (cp >> 6)); out[1] = (char)(0x80 | (cp & 0x3F)); out[2] = 0; }
}

/* merges of the synthetic vocabulary (left, right), in rank order; "\x20" is written as its symbol */
static const char *const SYN_MERGES[][2] = {
    { "t", "h" }, { "th", "e" }, { " ", "t" }, { "e", "r" }, { "i", "n" }, { "o", "n" },
    { "a", "n" }, { " ", "a" }, { " t", "he" }, { "e", "s" }, { "o", "r" }, { "l", "l" },
};
#define N_SYN_MERGES (sizeof SYN_MERGES / sizeof SYN_MERGES[0])

/* a piece of a merge as vocabulary text: every byte as its symbol */
static void syn_text(const char *piece, char *out, size_t cap)
{
    size_t n = 0;
    for (const unsigned char *c = (const unsigned char *)piece; *c && n + 3 < cap; c++) {
        char sym[4];
        byte_symbol(*c, sym);
        for (const char *q = sym; *q; q++) out[n++] = *q;
    }
    out[n] = 0;
}

static void syn_token(const qwen_synth_spec_t *s, uint32_t id, char *out, size_t cap)
{
    if (id < 256) { byte_symbol((int)id, out); return; }
    if (id < 256 + N_SYN_MERGES) {
        char l[32], r[32];
        syn_text(SYN_MERGES[id - 256][0], l, sizeof l);
        syn_text(SYN_MERGES[id - 256][1], r, sizeof r);
        snprintf(out, cap, "%s%s", l, r);
        return;
    }
    if (id == s->vocab - 3) { snprintf(out, cap, "<|endoftext|>"); return; }
    if (id == s->vocab - 2) { snprintf(out, cap, "<|im_start|>"); return; }
    if (id == s->vocab - 1) { snprintf(out, cap, "<|im_end|>"); return; }
    snprintf(out, cap, "<|t%u|>", id);
}

static int write_tokenizer(FILE *f, const qwen_synth_spec_t *s)
{
    int err = w_str(f, "tokenizer.ggml.model") | w_u32(f, GGUF_TYPE_STRING) | w_str(f, "gpt2");
    err |= w_str(f, "tokenizer.ggml.tokens") | w_u32(f, GGUF_TYPE_ARRAY) | w_u32(f, GGUF_TYPE_STRING) |
           w_u64(f, s->vocab);
    for (uint32_t id = 0; id < s->vocab; id++) {
        char t[64];
        syn_token(s, id, t, sizeof t);
        err |= w_str(f, t);
    }
    err |= w_str(f, "tokenizer.ggml.merges") | w_u32(f, GGUF_TYPE_ARRAY) | w_u32(f, GGUF_TYPE_STRING) |
           w_u64(f, N_SYN_MERGES);
    for (size_t m = 0; m < N_SYN_MERGES; m++) {
        char l[32], r[32], t[72];
        syn_text(SYN_MERGES[m][0], l, sizeof l);
        syn_text(SYN_MERGES[m][1], r, sizeof r);
        snprintf(t, sizeof t, "%s %s", l, r);
        err |= w_str(f, t);
    }
    return err;
}

int qwen_synth_write_gguf(const qwen_synth_spec_t *s, const char *path)
{
    const char *A = "qwen35";
    const uint32_t nt = qwen_synth_count(s);
    if (s->tokenizer && s->vocab < 256 + N_SYN_MERGES + 3) return -1;
    FILE *f = fopen(path, "wb");
    if (!f) return -1;
    char k[128];
    int err = 0;
    const uint32_t n_kv = 20 + (s->tokenizer ? 3 : 0);
    err |= w_u32(f, GGUF_MAGIC) | w_u32(f, 3) | w_u64(f, nt) | w_u64(f, n_kv);
    err |= w_str(f, "general.architecture") | w_u32(f, GGUF_TYPE_STRING) | w_str(f, A);
    err |= kv_u32(f, "general.alignment", 32);
#define KU(SUF, V) do { snprintf(k, sizeof k, "%s.%s", A, SUF); err |= kv_u32(f, k, V); } while (0)
#define KF(SUF, V) do { snprintf(k, sizeof k, "%s.%s", A, SUF); err |= kv_f32(f, k, V); } while (0)
    KU("embedding_length", s->n_embd);
    KU("attention.head_count", s->n_head);
    KU("attention.head_count_kv", s->n_kv_head);
    KU("attention.key_length", s->head_dim);
    KU("block_count", s->n_layer + 1);
    KU("feed_forward_length", s->n_ff);
    KU("vocab_size", s->vocab);
    KU("context_length", s->context_len);
    KF("rope.freq_base", s->rope_theta);
    KU("rope.dimension_count", s->rope_dim);
    KF("attention.layer_norm_rms_epsilon", s->eps);
    KU("full_attention_interval", s->full_attn_interval);
    KU("ssm.state_size", s->state);
    KU("ssm.conv_kernel", 4);
    KU("ssm.inner_size", s->n_v_heads * s->state);
    KU("ssm.group_count", s->n_k_heads);
    KU("nextn_predict_layers", 1);
    snprintf(k, sizeof k, "%s.rope.dimension_sections", A);
    {
        const uint32_t secs[4] = { 11, 11, 10, 0 };
        err |= w_str(f, k) | w_u32(f, GGUF_TYPE_ARRAY) | w_u32(f, GGUF_TYPE_UINT32) | w_u64(f, 4);
        err |= w_bytes(f, secs, sizeof secs);
    }
    if (s->tokenizer) err |= write_tokenizer(f, s);
#undef KU
#undef KF
    uint64_t off = 0;
    for (uint32_t i = 0; i < nt; i++) {
        qwen_synth_tensor_t t;
        qwen_synth_describe(s, i, &t);
        err |= w_str(f, t.name) | w_u32(f, t.n_dims);
        for (uint32_t d = 0; d < t.n_dims; d++) err |= w_u64(f, t.ne[d]);
        err |= w_u32(f, (uint32_t)t.type) | w_u64(f, off);
        off += (t.nbytes + 31) / 32 * 32;
    }
    static const uint8_t zeros[32];
    long pos = ftell(f);
    err |= w_bytes(f, zeros, (size_t)((32 - pos % 32) % 32));
    for (uint32_t i = 0; i < nt && !err; i++) {
        qwen_synth_tensor_t t;
        qwen_synth_describe(s, i, &t);
        void *buf = malloc(t.nbytes ? t.nbytes : 1);
        if (!buf || qwen_synth_fill(s, i, buf)) { free(buf); err = 1; break; }
        err |= w_bytes(f, buf, t.nbytes);
        err |= w_bytes(f, zeros, (size_t)((32 - t.nbytes % 32) % 32));
        free(buf);
    }
    if (fclose(f)) err = 1;
    return err ? -1 : 0;
}
