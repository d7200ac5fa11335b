/*
 * or_model.c -- oracle restatement of the reference model runtime and spec
 * driver: GGUF reader (reference src/gguf.c:84-317), model_init
 * (src/model.c:55-290), gated attention (src/model.c:318-485,760-843),
 * Gated DeltaNet (src/model.c:494-695,845-974), forward / batched forward /
 * rollback / MTP (src/model.c:714-1103) and the greedy spec cycle
 * (src/main.c:133-231).  Test infrastructure only (see oracle.h).
 *
 * Generalisation beyond the reference: the number of checkpoint slots is
 * k_max instead of the compile-time SPEC_MAX_B-1 = 2 (include/model.h:113);
 * with k_max = 2 every code path is the reference's.
 */
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ====================== GGUF reader (gguf.c) ====================== */
typedef struct { const uint8_t *p, *end; } cur_t;

static int rdb(cur_t *c, void *dst, size_t n)            /* gguf.c:35-40 */
{
    if (n > (size_t)(c->end - c->p)) return -1;
    memcpy(dst, c->p, n);
    c->p += n;
    return 0;
}
static int rdstr(cur_t *c, char *dst, size_t max)        /* gguf.c:42-52 */
{
    uint64_t len;
    if (rdb(c, &len, 8) || len > (uint64_t)(c->end - c->p)) return -1;
    size_t k = len < max - 1 ? (size_t)len : max - 1;
    memcpy(dst, c->p, k);
    dst[k] = 0;
    c->p += len;
    return 0;
}
static size_t vsize(uint32_t t)                          /* gguf.c:14-29 */
{
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}
static int skipv(cur_t *c, uint32_t t)                   /* gguf.c:55-79 */
{
    if (t == 8) {
        uint64_t len;
        if (rdb(c, &len, 8) || len > (uint64_t)(c->end - c->p)) return -1;
        c->p += len;
        return 0;
    }
    if (t == 9) {
        uint32_t et; uint64_t cnt;
        if (rdb(c, &et, 4) || rdb(c, &cnt, 8) || et > 12) return -1;
        for (uint64_t i = 0; i < cnt; i++) if (skipv(c, et)) return -1;
        return 0;
    }
    uint8_t tmp[8];
    return rdb(c, tmp, vsize(t));
}

typedef struct {
    void *map; size_t size; uint32_t align; char arch[32];
    uint64_t n_kv, n_tensors;
    or_config_t cfg;
    or_tensor_t *tensors;
} gguf_t;

/* gguf.c:84-170 : two passes, "<arch>.<suffix>" keys with exact types */
static int parse_kv(gguf_t *g, cur_t *c, int pass)
{
    struct { const char *suf; uint32_t type; void *dst; } f[] = {
        { ".embedding_length", 4, &g->cfg.n_embd },
        { ".attention.head_count", 4, &g->cfg.n_head },
        { ".attention.head_count_kv", 4, &g->cfg.n_head_kv },
        { ".attention.key_length", 4, &g->cfg.head_dim },
        { ".block_count", 4, &g->cfg.n_layer },
        { ".feed_forward_length", 4, &g->cfg.n_ff },
        { ".vocab_size", 4, &g->cfg.vocab_size },
        { ".context_length", 4, &g->cfg.context_len },
        { ".rope.freq_base", 6, &g->cfg.rope_theta },
        { ".rope.dimension_count", 4, &g->cfg.rope_dim_count },
        { ".attention.layer_norm_rms_epsilon", 6, &g->cfg.rms_norm_eps },
        { ".full_attention_interval", 4, &g->cfg.full_attn_interval },
        { ".ssm.state_size", 4, &g->cfg.ssm_state_size },
        { ".ssm.conv_kernel", 4, &g->cfg.ssm_conv_kernel },
        { ".ssm.inner_size", 4, &g->cfg.ssm_inner_size },
        { ".ssm.group_count", 4, &g->cfg.ssm_group_count },
        { ".nextn_predict_layers", 4, &g->cfg.nextn_layers },
    };
    for (uint64_t i = 0; i < g->n_kv; i++) {
        char key[160]; uint32_t t;
        if (rdstr(c, key, sizeof key) || rdb(c, &t, 4) || t > 12) return -1;
        if (pass == 1) {
            if (!strcmp(key, "general.architecture") && t == 8) {
                if (rdstr(c, g->arch, sizeof g->arch)) return -1;
                continue;
            }
            if (!strcmp(key, "general.alignment") && t == 4) {
                uint32_t a;
                if (rdb(c, &a, 4)) return -1;
                if (a) g->align = a;
                continue;
            }
            if (skipv(c, t)) return -1;
            continue;
        }
        char want[192];
        snprintf(want, sizeof want, "%s.rope.dimension_sections", g->arch);
        if (!strcmp(key, want) && t == 9) {
            uint32_t et; uint64_t cnt;
            if (rdb(c, &et, 4) || rdb(c, &cnt, 8) || (et != 4 && et != 5)) return -1;
            for (uint64_t k = 0; k < cnt; k++) {
                uint32_t v;
                if (rdb(c, &v, 4)) return -1;
                if (k < 4) g->cfg.rope_sections[k] = v;
            }
            continue;
        }
        int used = 0;
        for (size_t j = 0; j < sizeof f / sizeof f[0] && !used; j++) {
            snprintf(want, sizeof want, "%s%s", g->arch, f[j].suf);
            if (!strcmp(key, want) && t == f[j].type) {
                if (rdb(c, f[j].dst, 4)) return -1;
                used = 1;
            }
        }
        if (!used && skipv(c, t)) return -1;
    }
    return 0;
}

static void gguf_free(gguf_t *g)
{
    if (g->map) munmap(g->map, g->size);
    free(g->tensors);
    memset(g, 0, sizeof *g);
}

/* gguf.c:185-310 */
static int gguf_load(gguf_t *g, const char *path)
{
    memset(g, 0, sizeof *g);
    g->align = 32;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return -1;
    struct stat st;
    if (fstat(fd, &st) || st.st_size < 24) { close(fd); return -1; }
    g->size = (size_t)st.st_size;
    g->map = mmap(NULL, g->size, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) { g->map = NULL; return -1; }
    cur_t c = { (const uint8_t *)g->map, (const uint8_t *)g->map + g->size };
    uint32_t magic, ver;
    if (rdb(&c, &magic, 4) || rdb(&c, &ver, 4) || rdb(&c, &g->n_tensors, 8) || rdb(&c, &g->n_kv, 8))
        goto fail;
    if (magic != 0x46554747u || ver < 2 || ver > 3) goto fail;
    const uint8_t *kv0 = c.p;
    if (parse_kv(g, &c, 1) || !g->arch[0]) goto fail;
    c.p = kv0;
    if (parse_kv(g, &c, 2)) goto fail;
    if (g->n_tensors == 0 || g->n_tensors > 100000) goto fail;
    g->tensors = (or_tensor_t *)calloc(g->n_tensors, sizeof *g->tensors);
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        or_tensor_t *t = &g->tensors[i];
        uint32_t type;
        if (rdstr(&c, t->name, sizeof t->name) || rdb(&c, &t->n_dims, 4) || t->n_dims > 4) goto fail;
        for (uint32_t d = 0; d < t->n_dims; d++) if (rdb(&c, &t->ne[d], 8)) goto fail;
        if (rdb(&c, &type, 4) || rdb(&c, &t->offset, 8)) goto fail;
        t->type = (int)type;
    }
    uint64_t pos = (uint64_t)(c.p - (const uint8_t *)g->map);
    uint64_t base = (pos + g->align - 1) / g->align * g->align;
    if (base >= g->size) goto fail;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        g->tensors[i].data = (const uint8_t *)g->map + base + g->tensors[i].offset;
        if ((const uint8_t *)g->tensors[i].data >= c.end) goto fail;
    }
    if (g->cfg.vocab_size == 0)
        for (uint64_t i = 0; i < g->n_tensors; i++)
            if (!strcmp(g->tensors[i].name, "token_embd.weight") && g->tensors[i].n_dims == 2)
                g->cfg.vocab_size = (uint32_t)g->tensors[i].ne[1];
    return 0;
fail:
    gguf_free(g);
    return -1;
}

static const or_tensor_t *find(const gguf_t *g, const char *name)   /* gguf.c:312-317 */
{
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (!strcmp(g->tensors[i].name, name)) return &g->tensors[i];
    return NULL;
}

/* ====================== model (model.c) ====================== */
typedef struct {
    int rec, ir;
    const or_tensor_t *attn_norm, *post_norm, *ffn_gate, *ffn_up, *ffn_down;
    const or_tensor_t *q, *k, *v, *q_norm, *k_norm, *o;
    const or_tensor_t *wqkv, *wgate, *conv1d, *dt_bias, *ssm_a, *beta, *alpha, *ssm_norm, *ssm_out;
    float *kv_k, *kv_v, *conv, *ssm;
} layer_t;

struct or_model {
    gguf_t g;
    or_config_t cfg;
    uint32_t n_embd, n_ff, n_layer, n_head, n_kv, hd, n_v, n_k, hk, hv, d_inner, conv_dim;
    uint32_t n_recr, n_attn, n_ctx, pos, k_max, specb;
    float eps;
    layer_t *L, mtp;
    const or_tensor_t *tok_embd, *out_norm, *output, *eh_proj, *enorm, *hnorm, *shnorm;
    float *x, *xb, *qkv, *kvs, *z, *ffn, *attn, *logits, *scores, *rope_cos, *rope_sin;
    float *bx, *bxb, *bqkv, *bkv, *bz, *bffn, *battn, *h_save, *logits_b, *mtp_h;
    float *ckpt_conv, *ckpt_ssm;
    int nthreads;
};

#define F32(t) ((const float *)(t)->data)
static float *zalloc(size_t n) { return (float *)calloc(n ? n : 1, sizeof(float)); }

static void gemv_b(or_model_t *m, const or_tensor_t *W, const float *x, uint64_t ldx, int n,
                   float *out, uint64_t ldo)
{
    or_gemv_batch(W->type, W->data, W->ne[0], W->ne[1], x, ldx, n, out, ldo, m->nthreads);
}
static void gemv1(or_model_t *m, const or_tensor_t *W, const float *x, float *out)
{
    gemv_b(m, W, x, W->ne[0], 1, out, W->ne[1]);
}

static int chk2(const or_tensor_t *t, uint64_t a, uint64_t b)        /* model.c:37-44 */
{
    return !t || t->n_dims != 2 || t->ne[0] != a || t->ne[1] != b;
}
static int chk1(const or_tensor_t *t, uint64_t a)                    /* model.c:46-53 */
{
    return !t || t->n_dims != 1 || t->ne[0] != a;
}

void or_model_close(or_model_t *m)
{
    if (!m) return;
    if (m->L)
        for (uint32_t i = 0; i < m->n_layer; i++) {
            free(m->L[i].kv_k); free(m->L[i].kv_v); free(m->L[i].conv); free(m->L[i].ssm);
        }
    free(m->L);
    free(m->mtp.kv_k); free(m->mtp.kv_v);
    float *bufs[] = { m->x, m->xb, m->qkv, m->kvs, m->z, m->ffn, m->attn, m->logits, m->scores,
                      m->rope_cos, m->rope_sin, m->bx, m->bxb, m->bqkv, m->bkv, m->bz, m->bffn,
                      m->battn, m->h_save, m->logits_b, m->mtp_h, m->ckpt_conv, m->ckpt_ssm };
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) free(bufs[i]);
    gguf_free(&m->g);
    free(m);
}

/* model.c:55-290 */
or_model_t *or_model_open(const char *path, uint32_t n_ctx, uint32_t k_max)
{
    or_model_t *m = (or_model_t *)calloc(1, sizeof *m);
    if (gguf_load(&m->g, path)) { free(m); return NULL; }
    m->cfg = m->g.cfg;
    const or_config_t *c = &m->cfg;
    m->nthreads = 1;
    m->n_embd = c->n_embd; m->n_ff = c->n_ff; m->n_head = c->n_head; m->n_kv = c->n_head_kv;
    m->hd = c->head_dim; m->n_k = c->ssm_group_count; m->hk = m->hv = c->ssm_state_size;
    m->d_inner = c->ssm_inner_size; m->eps = c->rms_norm_eps;
    m->k_max = k_max ? k_max : 1;
    m->specb = m->k_max + 1;
    const or_tensor_t *a0 = find(&m->g, "blk.0.ssm_a");
    if (!a0 || a0->n_dims != 1) goto fail;
    m->n_v = (uint32_t)a0->ne[0];
    m->conv_dim = 2 * m->n_k * m->hk + m->d_inner;
    m->n_layer = c->n_layer > c->nextn_layers ? c->n_layer - c->nextn_layers : c->n_layer;
    if (m->d_inner != m->n_v * m->hv || m->n_v > 256 || m->hv > 256 || m->hk > 256) goto fail;
    m->tok_embd = find(&m->g, "token_embd.weight");
    m->out_norm = find(&m->g, "output_norm.weight");
    m->output = find(&m->g, "output.weight");
    if (!m->output) m->output = m->tok_embd;
    if (!m->tok_embd || !m->out_norm || chk2(m->tok_embd, m->n_embd, c->vocab_size)) goto fail;

    m->L = (layer_t *)calloc(m->n_layer, sizeof(layer_t));
    char nm[96];
#define GET(field, fmt) do { snprintf(nm, sizeof nm, fmt, il); if (!(Ly->field = find(&m->g, nm))) goto fail; } while (0)
    for (uint32_t il = 0; il < m->n_layer; il++) {
        layer_t *Ly = &m->L[il];
        Ly->rec = ((il + 1) % c->full_attn_interval) != 0;
        GET(attn_norm, "blk.%u.attn_norm.weight");
        GET(post_norm, "blk.%u.post_attention_norm.weight");
        GET(ffn_gate, "blk.%u.ffn_gate.weight");
        GET(ffn_up, "blk.%u.ffn_up.weight");
        GET(ffn_down, "blk.%u.ffn_down.weight");
        if (chk2(Ly->ffn_gate, m->n_embd, m->n_ff) || chk2(Ly->ffn_up, m->n_embd, m->n_ff) ||
            chk2(Ly->ffn_down, m->n_ff, m->n_embd)) goto fail;
        if (Ly->rec) {
            GET(wqkv, "blk.%u.attn_qkv.weight"); GET(wgate, "blk.%u.attn_gate.weight");
            GET(conv1d, "blk.%u.ssm_conv1d.weight"); GET(dt_bias, "blk.%u.ssm_dt.bias");
            GET(ssm_a, "blk.%u.ssm_a"); GET(beta, "blk.%u.ssm_beta.weight");
            GET(alpha, "blk.%u.ssm_alpha.weight"); GET(ssm_norm, "blk.%u.ssm_norm.weight");
            GET(ssm_out, "blk.%u.ssm_out.weight");
            if (chk2(Ly->wqkv, m->n_embd, m->conv_dim) || chk2(Ly->wgate, m->n_embd, m->d_inner) ||
                chk2(Ly->conv1d, c->ssm_conv_kernel, m->conv_dim) || chk2(Ly->beta, m->n_embd, m->n_v) ||
                chk2(Ly->alpha, m->n_embd, m->n_v) || chk2(Ly->ssm_out, m->d_inner, m->n_embd) ||
                chk1(Ly->dt_bias, m->n_v) || chk1(Ly->ssm_a, m->n_v) || chk1(Ly->ssm_norm, m->hv)) goto fail;
            Ly->ir = (int)m->n_recr++;
        } else {
            GET(q, "blk.%u.attn_q.weight"); GET(k, "blk.%u.attn_k.weight"); GET(v, "blk.%u.attn_v.weight");
            GET(q_norm, "blk.%u.attn_q_norm.weight"); GET(k_norm, "blk.%u.attn_k_norm.weight");
            GET(o, "blk.%u.attn_output.weight");
            if (chk2(Ly->q, m->n_embd, 2 * m->n_head * m->hd) || chk2(Ly->k, m->n_embd, m->n_kv * m->hd) ||
                chk2(Ly->v, m->n_embd, m->n_kv * m->hd) || chk2(Ly->o, m->n_head * m->hd, m->n_embd) ||
                chk1(Ly->q_norm, m->hd) || chk1(Ly->k_norm, m->hd)) goto fail;
            m->n_attn++;
        }
    }
    m->n_ctx = n_ctx;
    const size_t kv = (size_t)n_ctx * m->n_kv * m->hd, cs = (size_t)m->conv_dim * 4,
                 ss = (size_t)m->n_v * m->hv * m->hk;
    for (uint32_t il = 0; il < m->n_layer; il++) {
        if (m->L[il].rec) { m->L[il].conv = zalloc(cs); m->L[il].ssm = zalloc(ss); }
        else { m->L[il].kv_k = zalloc(kv); m->L[il].kv_v = zalloc(kv); }
    }
    size_t sq = m->conv_dim;
    if (2 * m->n_head * m->hd > sq) sq = 2 * m->n_head * m->hd;
    if (m->n_ff > sq) sq = m->n_ff;
    m->x = zalloc(m->n_embd); m->xb = zalloc(m->n_embd); m->qkv = zalloc(sq);
    m->kvs = zalloc(2 * m->n_kv * m->hd); m->z = zalloc(m->d_inner); m->ffn = zalloc(m->n_ff);
    m->attn = zalloc(m->n_head * m->hd > m->d_inner ? m->n_head * m->hd : m->d_inner);
    m->logits = zalloc(c->vocab_size); m->scores = zalloc((size_t)m->n_head * n_ctx);
    /* model.c:186-201 RoPE tables */
    const uint32_t half = c->rope_dim_count / 2;
    m->rope_cos = zalloc((size_t)n_ctx * half); m->rope_sin = zalloc((size_t)n_ctx * half);
    for (uint32_t p = 0; p < n_ctx; p++)
        for (uint32_t i = 0; i < half; i++) {
            float ang = (float)p * powf(c->rope_theta, -2.0f * (float)i / (float)c->rope_dim_count);
            m->rope_cos[(size_t)p * half + i] = cosf(ang);
            m->rope_sin[(size_t)p * half + i] = sinf(ang);
        }
    /* model.c:203-230 batch arenas (B <= 8, stride n_ff) */
    const size_t B = 8;
    m->bx = zalloc(B * m->n_embd); m->bxb = zalloc(B * m->n_embd); m->bqkv = zalloc(B * m->n_ff);
    m->bkv = zalloc(B * 2 * m->n_kv * m->hd); m->bz = zalloc(B * m->d_inner);
    m->bffn = zalloc(B * m->n_ff);
    m->battn = zalloc(B * (m->n_head * m->hd > m->d_inner ? m->n_head * m->hd : m->d_inner));
    m->h_save = zalloc(B * m->n_embd);
    m->logits_b = zalloc(B * (size_t)c->vocab_size); m->mtp_h = zalloc(m->n_embd);
    /* model.c:232-237 checkpoints: k_max slots (reference: SPEC_MAX_B-1) */
    m->ckpt_conv = zalloc((size_t)m->k_max * m->n_recr * cs);
    m->ckpt_ssm = zalloc((size_t)m->k_max * m->n_recr * ss);
    /* model.c:239-284 MTP layer blk.{n_layer} */
    {
        layer_t *Ly = &m->mtp;
        const uint32_t il = m->n_layer;
        GET(attn_norm, "blk.%u.attn_norm.weight"); GET(post_norm, "blk.%u.post_attention_norm.weight");
        GET(q, "blk.%u.attn_q.weight"); GET(k, "blk.%u.attn_k.weight"); GET(v, "blk.%u.attn_v.weight");
        GET(q_norm, "blk.%u.attn_q_norm.weight"); GET(k_norm, "blk.%u.attn_k_norm.weight");
        GET(o, "blk.%u.attn_output.weight"); GET(ffn_gate, "blk.%u.ffn_gate.weight");
        GET(ffn_up, "blk.%u.ffn_up.weight"); GET(ffn_down, "blk.%u.ffn_down.weight");
        snprintf(nm, sizeof nm, "blk.%u.nextn.eh_proj.weight", il); m->eh_proj = find(&m->g, nm);
        snprintf(nm, sizeof nm, "blk.%u.nextn.enorm.weight", il); m->enorm = find(&m->g, nm);
        snprintf(nm, sizeof nm, "blk.%u.nextn.hnorm.weight", il); m->hnorm = find(&m->g, nm);
        snprintf(nm, sizeof nm, "blk.%u.nextn.shared_head_norm.weight", il); m->shnorm = find(&m->g, nm);
        if (chk2(m->eh_proj, 2 * m->n_embd, m->n_embd) || chk1(m->enorm, m->n_embd) ||
            chk1(m->hnorm, m->n_embd) || chk1(m->shnorm, m->n_embd)) goto fail;
        Ly->kv_k = zalloc(kv); Ly->kv_v = zalloc(kv);
    }
#undef GET
    return m;
fail:
    or_model_close(m);
    return NULL;
}

const or_config_t *or_model_config(const or_model_t *m) { return &m->cfg; }
int or_model_n_layer(const or_model_t *m) { return (int)m->n_layer; }
int or_model_n_embd(const or_model_t *m) { return (int)m->n_embd; }
uint32_t or_model_vocab(const or_model_t *m) { return m->cfg.vocab_size; }
uint32_t or_model_pos(const or_model_t *m) { return m->pos; }
void or_model_set_pos(or_model_t *m, uint32_t p) { m->pos = p; }
float *or_model_logits(or_model_t *m) { return m->logits; }
float *or_model_logits_b(or_model_t *m) { return m->logits_b; }
float *or_model_h_save(or_model_t *m) { return m->h_save; }
float *or_model_mtp_h(or_model_t *m) { return m->mtp_h; }
float *or_model_x(or_model_t *m) { return m->x; }
void or_model_set_threads(or_model_t *m, int n) { m->nthreads = n < 1 ? 1 : n; }
float *or_model_ssm_state(or_model_t *m, int ir)
{
    for (uint32_t i = 0; i < m->n_layer; i++) if (m->L[i].rec && m->L[i].ir == ir) return m->L[i].ssm;
    return NULL;
}
float *or_model_conv_state(or_model_t *m, int ir)
{
    for (uint32_t i = 0; i < m->n_layer; i++) if (m->L[i].rec && m->L[i].ir == ir) return m->L[i].conv;
    return NULL;
}

static float dot8(const float *a, const float *b, uint32_t n)   /* 8-lane FMA dot + hsum256 */
{
    float acc[8] = {0};
    for (uint32_t i = 0; i < n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    const float L0 = acc[0] + acc[4], L1 = acc[1] + acc[5], L2 = acc[2] + acc[6], L3 = acc[3] + acc[7];
    return (L0 + L1) + (L2 + L3);
}

/* model.c:323-333 NeoX partial RoPE: pairs (i, i+half) over the first rope_dim_count dims */
static void rope(const or_model_t *m, float *v, uint32_t pos)
{
    const uint32_t half = m->cfg.rope_dim_count / 2;
    const float *cs = m->rope_cos + (size_t)pos * half, *sn = m->rope_sin + (size_t)pos * half;
    for (uint32_t i = 0; i < half; i++) {
        const float v0 = v[i], v1 = v[i + half];
        v[i] = v0 * cs[i] - v1 * sn[i];
        v[i + half] = v0 * sn[i] + v1 * cs[i];
    }
}

/* model.c:353-406 per-head scores -> softmax -> V accumulation -> sigmoid gate */
static void attn_heads(or_model_t *m, layer_t *Ly, float *qkv, uint64_t ldx, float *out,
                       uint64_t ostride, uint32_t pos, uint32_t B)
{
    const uint32_t hd = m->hd, kvrow = m->n_kv * hd, per = m->n_head / m->n_kv;
    const float sc = 1.0f / sqrtf((float)hd);
    for (uint32_t h = 0; h < m->n_head; h++) {
        const uint32_t kh = h / per;
        float *s = m->scores + (size_t)h * m->n_ctx;
        for (uint32_t b = 0; b < B; b++) {
            float *qh = qkv + (size_t)b * ldx + h * 2 * hd, *gate = qh + hd;
            float *oh = out + (size_t)b * ostride + h * hd;
            const uint32_t pl = pos + b;
            for (uint32_t t = 0; t <= pl; t++)
                s[t] = dot8(qh, Ly->kv_k + (size_t)t * kvrow + kh * hd, hd) * sc;
            or_softmax_inplace(s, pl + 1);
            memset(oh, 0, hd * sizeof(float));
            for (uint32_t t = 0; t <= pl; t++) {
                const float *vt = Ly->kv_v + (size_t)t * kvrow + kh * hd;
                for (uint32_t i = 0; i < hd; i++) oh[i] = fmaf(s[t], vt[i], oh[i]);
            }
            or_sigmoid_inplace(gate, hd);
            for (uint32_t i = 0; i < hd; i++) oh[i] *= gate[i];
        }
    }
}

/* model.c:760-843 batched gated attention layer (B=1 equals model.c:418-485) */
static void attn_layer_b(or_model_t *m, layer_t *Ly, float *bx, float *bxb, float *bqkv,
                         float *bkv, float *battn, float *bffn, uint64_t stride,
                         uint32_t pos, uint32_t B)
{
    const uint32_t hd = m->hd, kvrow = m->n_kv * hd, ne = m->n_embd, nf = m->n_ff;
    for (uint32_t b = 0; b < B; b++) or_rmsnorm(bxb + b * ne, bx + b * ne, F32(Ly->attn_norm), ne, m->eps);
    gemv_b(m, Ly->q, bxb, ne, (int)B, bqkv, stride);
    gemv_b(m, Ly->k, bxb, ne, (int)B, bkv, 2 * kvrow);
    gemv_b(m, Ly->v, bxb, ne, (int)B, bkv + kvrow, 2 * kvrow);
    for (uint32_t b = 0; b < B; b++) {
        for (uint32_t h = 0; h < m->n_head; h++) {
            float *qh = bqkv + b * stride + h * 2 * hd;
            or_rmsnorm(qh, qh, F32(Ly->q_norm), hd, m->eps);
        }
        for (uint32_t kh = 0; kh < m->n_kv; kh++) {
            float *kp = bkv + b * 2 * kvrow + kh * hd;
            or_rmsnorm(kp, kp, F32(Ly->k_norm), hd, m->eps);
        }
        memcpy(Ly->kv_k + (size_t)(pos + b) * kvrow, bkv + b * 2 * kvrow, kvrow * sizeof(float));
        memcpy(Ly->kv_v + (size_t)(pos + b) * kvrow, bkv + b * 2 * kvrow + kvrow, kvrow * sizeof(float));
    }
    for (uint32_t b = 0; b < B; b++) {
        for (uint32_t h = 0; h < m->n_head; h++) rope(m, bqkv + b * stride + h * 2 * hd, pos + b);
        for (uint32_t kh = 0; kh < m->n_kv; kh++) rope(m, Ly->kv_k + (size_t)(pos + b) * kvrow + kh * hd, pos + b);
    }
    attn_heads(m, Ly, bqkv, stride, battn, m->n_head * hd, pos, B);
    gemv_b(m, Ly->o, battn, m->n_head * hd, (int)B, bxb, ne);
    for (uint32_t i = 0; i < B * ne; i++) bx[i] += bxb[i];
    for (uint32_t b = 0; b < B; b++) or_rmsnorm(bxb + b * ne, bx + b * ne, F32(Ly->post_norm), ne, m->eps);
    gemv_b(m, Ly->ffn_gate, bxb, ne, (int)B, bffn, nf);
    gemv_b(m, Ly->ffn_up, bxb, ne, (int)B, bqkv, stride);
    for (uint32_t b = 0; b < B; b++) or_silu_inplace(bffn + b * nf, nf);
    for (uint32_t b = 0; b < B; b++)
        for (uint32_t i = 0; i < nf; i++) bffn[b * nf + i] *= bqkv[b * stride + i];
    gemv_b(m, Ly->ffn_down, bffn, nf, (int)B, bxb, ne);
    for (uint32_t i = 0; i < B * ne; i++) bx[i] += bxb[i];
}

/* model.c:494-524 fused two-pass row update of one v-head state */
static void gdn_head(float *S, const float *q, const float *k, const float *v, float beta,
                     float decay, float kq, float qs, float *o, uint32_t hk, uint32_t hv)
{
    for (uint32_t j = 0; j < hk; j++) {
        float *row = S + (size_t)j * hv;
        const float delta = decay * dot8(row, k, hv);
        const float dj = (v[j] - delta) * beta;
        o[j] = (decay * dot8(row, q, hv) + dj * kq) * qs;
        for (uint32_t i = 0; i < hv; i++) row[i] = fmaf(dj, k[i], decay * row[i]);
    }
}

/* conv1d shift + 4 taps (model.c:891-903), SiLU (:909), per-k-head L2norm of q,k (:911-916) */
static void gdn_conv_token(int conv_dim, int n_k, int hk, float eps, float *xq,
                           float *state, const float *cw)
{
    for (int c = 0; c < conv_dim; c++) {
        float *s = state + c * 4;
        s[0] = s[1]; s[1] = s[2]; s[2] = s[3]; s[3] = xq[c];
        const float *w = cw + c * 4;
        xq[c] = s[0] * w[0] + s[1] * w[1] + s[2] * w[2] + s[3] * w[3];
    }
    or_silu_inplace(xq, (uint64_t)conv_dim);
    for (int kh = 0; kh < n_k; kh++) {
        or_l2norm(xq + kh * hk, xq + kh * hk, (uint64_t)hk, eps);
        or_l2norm(xq + n_k * hk + kh * hk, xq + n_k * hk + kh * hk, (uint64_t)hk, eps);
    }
}

/* model.c:558-587 one token of the recurrence over all v-heads (v-head h uses k-head h % n_k) */
static void gdn_ssm_token(int n_k, int n_v, int hk, int hv, const float *xq, const float *beta_r,
                          const float *alpha_r, const float *dt_bias, const float *ssm_a,
                          float *ssm, float *out)
{
    const float qs = 1.0f / sqrtf((float)hk);
    const size_t he = (size_t)hv * hk;
    for (int h = 0; h < n_v; h++) {
        const int kh = h % n_k;
        const float *q = xq + kh * hk, *k = xq + n_k * hk + kh * hk, *v = xq + 2 * n_k * hk + h * hv;
        const float b = 1.0f / (1.0f + expf(-beta_r[h]));
        const float ar = alpha_r[h] + dt_bias[h];
        const float sp = (ar > 30.0f) ? ar : log1pf(expf(ar));
        const float decay = expf(ssm_a[h] * sp);
        const float kq = dot8(k, q, (uint32_t)hk);
        gdn_head(ssm + (size_t)h * he, q, k, v, b, decay, kq, qs, out + h * hv, (uint32_t)hk, (uint32_t)hv);
    }
}

void or_gdn_block(int T, int conv_dim, int n_k, int n_v, int hk, int hv, float eps,
                  const float *qkv_raw, const float *beta_raw, const float *alpha_raw,
                  const float *conv_w, const float *dt_bias, const float *ssm_a,
                  float *conv_state, float *ssm_state, float *out,
                  float *snap_conv, float *snap_ssm)
{
    float *xq = zalloc((size_t)conv_dim);
    const size_t ss = (size_t)n_v * hv * hk;
    for (int b = 0; b < T; b++) {
        memcpy(xq, qkv_raw + (size_t)b * conv_dim, (size_t)conv_dim * sizeof(float));
        gdn_conv_token(conv_dim, n_k, hk, eps, xq, conv_state, conv_w);
        if (snap_conv) memcpy(snap_conv + (size_t)b * conv_dim * 4, conv_state, (size_t)conv_dim * 4 * sizeof(float));
        gdn_ssm_token(n_k, n_v, hk, hv, xq, beta_raw + (size_t)b * n_v, alpha_raw + (size_t)b * n_v,
                      dt_bias, ssm_a, ssm_state, out + (size_t)b * n_v * hv);
        if (snap_ssm) memcpy(snap_ssm + (size_t)b * ss, ssm_state, ss * sizeof(float));
    }
    free(xq);
}

/* model.c:845-974 batched GDN layer (B=1 with ckpt=0 equals model.c:617-695) */
static void gdn_layer_b(or_model_t *m, layer_t *Ly, uint32_t B, int ckpt)
{
    const uint32_t ne = m->n_embd, nf = m->n_ff, cd = m->conv_dim, di = m->d_inner, st = m->n_ff;
    float beta[8][256], alpha[8][256];
    for (uint32_t b = 0; b < B; b++) or_rmsnorm(m->bxb + b * ne, m->bx + b * ne, F32(Ly->attn_norm), ne, m->eps);
    gemv_b(m, Ly->wqkv, m->bxb, ne, (int)B, m->bqkv, st);
    gemv_b(m, Ly->wgate, m->bxb, ne, (int)B, m->bz, di);
    gemv_b(m, Ly->beta, m->bxb, ne, (int)B, &beta[0][0], 256);
    gemv_b(m, Ly->alpha, m->bxb, ne, (int)B, &alpha[0][0], 256);
    const uint32_t n_ckpt = B < m->specb ? B : m->specb;
    const size_t cs = (size_t)cd * 4, ss = (size_t)m->n_v * m->hv * m->hk;
    for (uint32_t b = 0; b < B; b++) {
        gdn_conv_token((int)cd, (int)m->n_k, (int)m->hk, m->eps, m->bqkv + b * st, Ly->conv, F32(Ly->conv1d));
        if (ckpt && b + 1 < n_ckpt)
            memcpy(m->ckpt_conv + (size_t)b * m->n_recr * cs + (size_t)Ly->ir * cs, Ly->conv, cs * sizeof(float));
    }
    for (uint32_t b = 0; b < B; b++) {
        gdn_ssm_token((int)m->n_k, (int)m->n_v, (int)m->hk, (int)m->hv, m->bqkv + b * st, beta[b],
                      alpha[b], F32(Ly->dt_bias), F32(Ly->ssm_a), Ly->ssm, m->battn + b * di);
        if (ckpt && b + 1 < n_ckpt)
            memcpy(m->ckpt_ssm + (size_t)b * m->n_recr * ss + (size_t)Ly->ir * ss, Ly->ssm, ss * sizeof(float));
    }
    for (uint32_t b = 0; b < B; b++) or_silu_inplace(m->bz + b * di, di);
    for (uint32_t b = 0; b < B; b++)
        for (uint32_t h = 0; h < m->n_v; h++) {
            float *o = m->battn + b * di + h * m->hv;
            const float *zh = m->bz + b * di + h * m->hv;
            or_rmsnorm(o, o, F32(Ly->ssm_norm), m->hv, m->eps);
            for (uint32_t i = 0; i < m->hv; i++) o[i] *= zh[i];
        }
    gemv_b(m, Ly->ssm_out, m->battn, di, (int)B, m->bxb, ne);
    for (uint32_t i = 0; i < B * ne; i++) m->bx[i] += m->bxb[i];
    for (uint32_t b = 0; b < B; b++) or_rmsnorm(m->bxb + b * ne, m->bx + b * ne, F32(Ly->post_norm), ne, m->eps);
    gemv_b(m, Ly->ffn_gate, m->bxb, ne, (int)B, m->bffn, nf);
    gemv_b(m, Ly->ffn_up, m->bxb, ne, (int)B, m->bqkv, st);
    for (uint32_t b = 0; b < B; b++) or_silu_inplace(m->bffn + b * nf, nf);
    for (uint32_t b = 0; b < B; b++)
        for (uint32_t i = 0; i < nf; i++) m->bffn[b * nf + i] *= m->bqkv[b * st + i];
    gemv_b(m, Ly->ffn_down, m->bffn, nf, (int)B, m->bxb, ne);
    for (uint32_t i = 0; i < B * ne; i++) m->bx[i] += m->bxb[i];
}

/* model.c:976-1002 */
void or_model_forward_batch(or_model_t *m, const uint32_t *tok, uint32_t pos, uint32_t B, int ckpt)
{
    const uint32_t ne = m->n_embd;
    const size_t rb = or_row_bytes(m->tok_embd->type, ne);
    for (uint32_t b = 0; b < B; b++)
        or_dequant_row(m->tok_embd->type, (const uint8_t *)m->tok_embd->data + (size_t)tok[b] * rb, ne, m->bx + b * ne);
    for (uint32_t il = 0; il < m->n_layer; il++) {
        layer_t *Ly = &m->L[il];
        if (Ly->rec) gdn_layer_b(m, Ly, B, ckpt);
        else attn_layer_b(m, Ly, m->bx, m->bxb, m->bqkv, m->bkv, m->battn, m->bffn, m->n_ff, pos, B);
    }
    memcpy(m->h_save, m->bx, (size_t)B * ne * sizeof(float));
    for (uint32_t b = 0; b < B; b++) or_rmsnorm(m->bxb + b * ne, m->bx + b * ne, F32(m->out_norm), ne, m->eps);
    gemv_b(m, m->output, m->bxb, ne, (int)B, m->logits_b, m->cfg.vocab_size);
    m->pos = pos + B;
}

/* model.c:714-744 : single-token step on the single-token buffers.  The
 * single-token layer code performs the same operations in the same order as
 * the batched code with B=1 (model.c:617-695 vs :845-974, :418-485 vs :760-843),
 * so it is restated through the batched layers on the single-token buffers. */
void or_model_forward(or_model_t *m, uint32_t token, uint32_t pos)
{
    const uint32_t ne = m->n_embd;
    const size_t rb = or_row_bytes(m->tok_embd->type, ne);
    or_dequant_row(m->tok_embd->type, (const uint8_t *)m->tok_embd->data + (size_t)token * rb, ne, m->x);
    /* run the layers through the batch path with B=1 and no checkpoints, using
     * the batch arenas as scratch; the residual lives in bx[0] for the pass */
    memcpy(m->bx, m->x, ne * sizeof(float));
    for (uint32_t il = 0; il < m->n_layer; il++) {
        layer_t *Ly = &m->L[il];
        if (Ly->rec) gdn_layer_b(m, Ly, 1, 0);
        else attn_layer_b(m, Ly, m->bx, m->bxb, m->bqkv, m->bkv, m->battn, m->bffn, m->n_ff, pos, 1);
    }
    memcpy(m->x, m->bx, ne * sizeof(float));
    or_rmsnorm(m->xb, m->x, F32(m->out_norm), ne, m->eps);
    gemv1(m, m->output, m->xb, m->logits);
    m->pos = pos + 1;
}

/* model.c:1015-1031 : restore all GDN states from checkpoint slot b */
void or_model_rollback_to(or_model_t *m, uint32_t b)
{
    const size_t cs = (size_t)m->conv_dim * 4, ss = (size_t)m->n_v * m->hv * m->hk;
    for (uint32_t il = 0; il < m->n_layer; il++) {
        layer_t *Ly = &m->L[il];
        if (!Ly->rec) continue;
        memcpy(Ly->conv, m->ckpt_conv + (size_t)b * m->n_recr * cs + (size_t)Ly->ir * cs, cs * sizeof(float));
        memcpy(Ly->ssm, m->ckpt_ssm + (size_t)b * m->n_recr * ss + (size_t)Ly->ir * ss, ss * sizeof(float));
    }
}

/* model.c:1038-1063 */
int or_mtp_forward(or_model_t *m, uint32_t token, uint32_t pos, int want_logits)
{
    const uint32_t ne = m->n_embd;
    const size_t rb = or_row_bytes(m->tok_embd->type, ne);
    float *cat = zalloc(2 * ne);
    or_dequant_row(m->tok_embd->type, (const uint8_t *)m->tok_embd->data + (size_t)token * rb, ne, cat);
    or_rmsnorm(cat, cat, F32(m->enorm), ne, m->eps);
    or_rmsnorm(cat + ne, m->mtp_h, F32(m->hnorm), ne, m->eps);
    gemv1(m, m->eh_proj, cat, m->x);
    free(cat);
    /* single-token gated attention layer on the MTP layer's own KV (model.c:1053 -> :418-485) */
    float *qkv = zalloc(m->n_ff > 2 * m->n_head * m->hd ? m->n_ff : 2 * m->n_head * m->hd);
    float *kvs = zalloc(2 * m->n_kv * m->hd);
    float *att = zalloc(m->n_head * m->hd);
    float *ffn = zalloc(m->n_ff);
    attn_layer_b(m, &m->mtp, m->x, m->xb, qkv, kvs, att, ffn,
                 m->n_ff > 2 * m->n_head * m->hd ? m->n_ff : 2 * m->n_head * m->hd, pos, 1);
    free(qkv); free(kvs); free(att); free(ffn);
    memcpy(m->mtp_h, m->x, ne * sizeof(float));
    if (want_logits) {
        or_rmsnorm(m->xb, m->x, F32(m->shnorm), ne, m->eps);
        gemv1(m, m->output, m->xb, m->logits);
    }
    return 0;
}

/* model.c:1069-1103 */
int or_mtp_forward_batch(or_model_t *m, const uint32_t *tok, uint32_t pos, uint32_t B, int want_logits)
{
    const uint32_t ne = m->n_embd, st = m->n_ff;
    const size_t rb = or_row_bytes(m->tok_embd->type, ne);
    for (uint32_t b = 0; b < B; b++) {
        float *cat = m->bqkv + (size_t)b * st;
        or_dequant_row(m->tok_embd->type, (const uint8_t *)m->tok_embd->data + (size_t)tok[b] * rb, ne, cat);
        or_rmsnorm(cat, cat, F32(m->enorm), ne, m->eps);
        or_rmsnorm(cat + ne, m->h_save + (size_t)b * ne, F32(m->hnorm), ne, m->eps);
    }
    gemv_b(m, m->eh_proj, m->bqkv, st, (int)B, m->bx, ne);
    attn_layer_b(m, &m->mtp, m->bx, m->bxb, m->bqkv, m->bkv, m->battn, m->bffn, st, pos, B);
    memcpy(m->mtp_h, m->bx + (size_t)(B - 1) * ne, ne * sizeof(float));
    if (want_logits) {
        for (uint32_t b = 0; b < B; b++) or_rmsnorm(m->bxb + b * ne, m->bx + b * ne, F32(m->shnorm), ne, m->eps);
        gemv_b(m, m->output, m->bxb, ne, (int)B, m->logits_b, m->cfg.vocab_size);
    }
    return 0;
}

/* main.c:133-152 : batched prefill in chunks of 8 (+ MTP prefill when drafting) */
static void prefill(or_model_t *m, const uint32_t *prompt, uint32_t n, int with_mtp)
{
    uint32_t pos = 0, last = 0;
    while (pos < n) {
        uint32_t B = n - pos > 8 ? 8 : n - pos;
        or_model_forward_batch(m, prompt + pos, pos, B, 0);
        if (with_mtp) or_mtp_forward_batch(m, prompt + pos, pos, B, 0);
        pos += B;
        last = B;
    }
    if (last)
        memcpy(m->logits, m->logits_b + (size_t)(last - 1) * m->cfg.vocab_size,
               (size_t)m->cfg.vocab_size * sizeof(float));
}

/* main.c:158-231 greedy MTP speculative decode.  force_accept (not in the
 * reference) fixes j: 1 = k every cycle (all drafts accepted), 2 = cycle index
 * mod (k + 1) (every rollback depth in turn). */
uint32_t or_generate_spec_ex(or_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                             uint32_t k_req, uint32_t eos, int force_accept, uint32_t *out, or_spec_stats_t *stt,
                             uint32_t *cycle_j)
{
    const uint32_t V = m->cfg.vocab_size, ne = m->n_embd;
    if (k_req > m->k_max) k_req = m->k_max;
    prefill(m, prompt, n_prompt, k_req > 0);
    uint32_t gen = 0;
    or_spec_stats_t s = {0, 0, 0};
    const float *last = m->logits;
    uint32_t cand[16];
    while (gen < n_predict) {
        const uint32_t P = m->pos - 1;
        const uint32_t room = m->n_ctx - 1 - P;
        if (room < 1) break;
        const uint32_t k = k_req < room - 1 ? k_req : room - 1;
        cand[0] = or_argmax(last, V);
        if (cand[0] == eos) break;
        for (uint32_t j = 1; j <= k; j++) {
            or_mtp_forward(m, cand[j - 1], P + j, 1);
            cand[j] = or_argmax(m->logits, V);
        }
        const uint32_t B = k + 1;
        or_model_forward_batch(m, cand, P + 1, B, 1);
        uint32_t j = k;
        if (force_accept == 2)
            j = (uint32_t)(s.n_cycles % (k + 1));
        else
            for (uint32_t i = 0; i < k && !force_accept; i++)
                if (or_argmax(m->logits_b + (size_t)i * V, V) != cand[i + 1]) { j = i; break; }
        for (uint32_t i = 0; i <= j && gen < n_predict; i++) out[gen++] = cand[i];
        if (cycle_j) cycle_j[s.n_cycles] = j;
        s.n_accepted += j;
        s.n_drafts += k;
        /* n_cycles counts every cycle run, also the one that reaches the context
         * end (main.c's printed counter skips that one) */
        if (m->pos >= m->n_ctx) { s.n_cycles++; break; }
        if (j < k) {
            or_model_rollback_to(m, j);
            m->pos = P + j + 2;
        }
        memcpy(m->mtp_h, m->h_save + (size_t)j * ne, ne * sizeof(float));
        or_mtp_forward(m, cand[j], P + j + 1, 0);
        last = m->logits_b + (size_t)j * V;
        s.n_cycles++;
    }
    if (stt) *stt = s;
    return gen;
}

uint32_t or_generate_spec(or_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                          uint32_t k, uint32_t eos, uint32_t *out, or_spec_stats_t *st, uint32_t *cycle_j)
{
    return or_generate_spec_ex(m, prompt, n_prompt, n_predict, k, eos, 0, out, st, cycle_j);
}

/* Plain greedy stream used as the lossless-spec oracle: argmax of model_forward
 * logits each step (debug_spec2.c:60-85 pattern; main.c:232-248 with temp <= 0
 * and no repeat penalty). */
/* main.c:232-248: prefill, then sample from the last logits, forward the sampled token,
 * sample again; the repeat penalty sees the prompt and every generated token
 * (all_tokens).  The sampler state advances in place. */
uint32_t or_generate_sample(or_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                            uint32_t eos, or_sampler_t *s, uint32_t *out)
{
    const uint32_t V = m->cfg.vocab_size;
    uint32_t *all = malloc(sizeof(uint32_t) * ((size_t)n_prompt + n_predict + 1));
    if (!all) return 0;
    memcpy(all, prompt, sizeof(uint32_t) * n_prompt);
    size_t n_all = n_prompt;
    prefill(m, prompt, n_prompt, 0);
    uint32_t cur = or_sampler_sample(s, m->logits, V, all, n_all), gen = 0;
    all[n_all++] = cur;
    out[gen++] = cur;
    for (uint32_t i = 1; i < n_predict; i++) {
        if (cur == eos || m->pos >= m->n_ctx) break;
        or_model_forward(m, cur, m->pos);
        cur = or_sampler_sample(s, m->logits, V, all, n_all);
        all[n_all++] = cur;
        out[gen++] = cur;
    }
    free(all);
    return gen;
}

uint32_t or_generate_greedy(or_model_t *m, const uint32_t *prompt, uint32_t n_prompt,
                            uint32_t n_predict, uint32_t eos, uint32_t *out)
{
    const uint32_t V = m->cfg.vocab_size;
    prefill(m, prompt, n_prompt, 0);
    uint32_t cur = or_argmax(m->logits, V), gen = 0;
    out[gen++] = cur;
    for (uint32_t i = 1; i < n_predict; i++) {
        if (cur == eos || m->pos >= m->n_ctx) break;
        or_model_forward(m, cur, m->pos);
        cur = or_argmax(m->logits, V);
        out[gen++] = cur;
    }
    return gen;
}
