/*
 * model.c -- the hybrid model on one MI355X behind the reference model.h API.
 *
 * Layer sequence per batched forward (B tokens, all buffers on the device):
 *   GDN  : rmsnorm -> grouped GEMV {qkv, gate, beta, alpha} -> conv1d+SiLU
 *          (snapshots) -> delta-rule recurrence (snapshots) -> gated rmsnorm
 *          -> ssm_out GEMV accumulated into the residual -> FFN
 *   attn : rmsnorm -> grouped GEMV {q, k, v} -> q/k norm + RoPE + KV write ->
 *          flash-decoding attention with sigmoid gate -> attn_out GEMV
 *          accumulated into the residual -> FFN
 *   FFN  : rmsnorm -> grouped GEMV {gate, up} -> silu(gate)*up -> down GEMV
 *          accumulated into the residual
 * The order of operations follows the reference model.c:714-1103; binding
 * and shape checks follow model.c:55-290.
 */
#define _POSIX_C_SOURCE 200809L
#include "model.h"
#include "qgpu.h"
#include "quant.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define NSLOT (SPEC_MAX_B + 1)      /* GDN state ring: current + one snapshot per batch token */
#define MAXB  SPEC_MAX_B

double qwen_prof_embed, qwen_prof_gdn, qwen_prof_attn, qwen_prof_head;
uint64_t qwen_prof_calls;

typedef struct {
    int rec;
    qgpu_tensor *ffn_gate, *ffn_up, *ffn_down, *q, *k, *v, *o, *wqkv, *wgate, *beta, *alpha, *ssm_out;
    float *attn_norm, *post_norm, *q_norm, *k_norm, *conv1d, *dt_bias, *ssm_a, *ssm_norm;
    float *kv_k, *kv_v;           /* attention: [n_ctx][n_kv*head_dim] */
    float *conv_ring, *ssm_ring;  /* GDN: NSLOT slots of conv (conv_dim*4) / ssm (n_v*128*128) state */
    float *gdn_f;                 /* GDN: two buffers of MAXB rank-1 factor records (f_tok floats each) */
} glayer_t;

struct qwen_gpu {
    glayer_t *L, mtp;
    qgpu_tensor *tok_embd, *output, *eh_proj;
    float *out_norm, *enorm, *hnorm, *shnorm, *rope_cos, *rope_sin;
    int *d_pos, *d_cur;
    /* embedding rows not yet in bx: the first preparation of the forward gathers them from
     * tok_embd (embd_fuse: packed IQ4_XS, n_embd % 256 == 0) */
    const uint32_t *pend_tok;
    uint32_t pend_tok_B;
    int embd_fuse;
    /* where the kernels of the next forward read the position and the ring slot: constant
     * tables d_posv[p] = p, d_curv[c] = c at host-chosen offsets for eager launches (no launch
     * sets them), or d_pos / d_cur, set before each captured-graph replay (see at()) */
    int *d_posv, *d_curv;
    const int *pos_ptr, *cur_ptr;
    uint32_t *d_tok, *d_cand, *d_vtok, *d_acc;
    /* the MTP re-anchor's token and hidden state, written by the acceptance kernel */
    uint32_t *anchor_tok;
    float *anchor_h;
    /* the acceptance result in pinned host memory (the kernel writes it, the host polls it) */
    uint32_t *h_acc;
    float *bx, *bxb, *bqkv, *bk, *bv, *bz, *bbeta, *balpha, *bffn, *battn, *xq, *h_save, *logits_b, *logits1,
          *mtp_h, *mx, *cat;
    uint64_t SQ, A, conv_elems, ssm_elems, kvrow;
    int cur, cur_base;
    int last_B;                 /* tokens of the last backbone forward: the states model_rollback_to may select */
    /* GDN factor form (qgpu_gdn_fused_factor), for forwards of factor_min_b tokens or more: the
     * state stays in the slot of the forward (fbase) and each token's rank-1 factors go to
     * factor buffer fpar; the next forward applies the (cur - fbase) % NSLOT kept tokens first.
     * fbase = -1: the states are snapshots (nothing pending).  fst_ptr: where the kernels read
     * {pending tokens, buffer}: the constant table d_fstv (eager) or d_fst (captured graphs). */
    int fbase, fpar, factor_min_b;
    uint64_t f_tok;
    int *d_fst, *d_fstv;
    const int *fst_ptr;
    /* K-split residual GEMVs leave partial planes (part, [ks][B][n_embd]) that the
     * next RMSNorm of that residual adds in (or materialize() when none follows) */
    float *part, *pend;
    int pend_ks;
    uint32_t pend_B;
    /* attention span blocks split a kv head's query heads while the live context of a B-token
     * forward is at most att_split[B] positions (qgpu_attn_split_bound; 0: never); att_live is
     * the bound the next body's attention launches are given (att_split[B] or 0) */
    int att_split[QGPU_MAX_B + 1], att_live;
    /* replayable launch sequences (HIP graphs) of the forward / MTP bodies, one per
     * (kind, token pointer, hidden-state pointer, logits pointer, B, flag, att_live) */
    int use_graphs, n_graphs;
    struct { int kind, flag, live; uint32_t B; const void *tok, *h, *lg; void *exec; } graphs[48];
    int status;               /* of the last call: 0, -1 rejected on the host, -2 device error */
    /* section timing of model_forward: events before the embedding, after it, after each layer
     * and after the head (n_layer + 3), recorded while prof_active */
    int prof, prof_active, n_pev;
    void **pev;
    void **allocs;
    size_t n_allocs, cap_allocs;
    qgpu_tensor **tensors;
    size_t n_tensors, cap_tensors;
};

static double now_s(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* The first device error is sticky: it is reported once, every later device
 * call is skipped, and the public entry points then do nothing (status -2).
 * A failed launch or a device fault leaves the HIP context unusable, so the
 * model stops rather than compute on it; the caller's process goes on. */
static int qwen_dev_err;

static void fail_rc(const char *what, int rc)
{
    if (!qwen_dev_err)
        fprintf(stderr, "qwen gpu: %s failed: %s (the model accepts no further calls)\n", what, qgpu_strerror(rc));
    qwen_dev_err = rc ? rc : -1;
}
#define K(call) do { if (!qwen_dev_err) { int _rc = (call); if (_rc) fail_rc(#call, _rc); } } while (0)

/* entry and exit of every public call: status 0 / -1 (rejected) / -2 (device error) */
static int call_begin(qwen_model_t *m)
{
    if (!m || !m->gpu) return -1;
    m->gpu->status = qwen_dev_err ? -2 : 0;
    return qwen_dev_err ? -1 : 0;
}
static void call_end(qwen_model_t *m)
{
    if (qwen_dev_err) m->gpu->status = -2;
}
static int reject(qwen_model_t *m, const char *fn, uint32_t pos, uint32_t B)
{
    fprintf(stderr, "%s: positions %u..%u outside the context (n_ctx = %u) or batch %u outside 1..%d; call ignored\n",
            fn, pos, pos + B - 1, m->n_ctx, B, SPEC_MAX_B);
    m->gpu->status = -1;
    return -1;
}
/* pos .. pos+B-1 must be KV rows of the cache (the device writes row pos+b) */
static int bad_span(const qwen_model_t *m, uint32_t pos, uint32_t B)
{
    return B < 1 || B > SPEC_MAX_B || pos >= m->n_ctx || B > m->n_ctx - pos;
}

/* ------------------------------------------------------------------ allocation */
static void *dalloc(qwen_gpu_t *g, size_t bytes)
{
    void *p = NULL;
    if (qgpu_malloc(&p, bytes ? bytes : 16)) return NULL;
    if (g->n_allocs == g->cap_allocs) {
        g->cap_allocs = g->cap_allocs ? 2 * g->cap_allocs : 256;
        g->allocs = realloc(g->allocs, g->cap_allocs * sizeof(void *));
    }
    g->allocs[g->n_allocs++] = p;
    qgpu_memset(p, 0, bytes ? bytes : 16);
    return p;
}

static void gpu_free(qwen_gpu_t *g)
{
    if (!g) return;
    qgpu_sync();
    for (int i = 0; i < g->n_graphs; i++) qgpu_graph_destroy(g->graphs[i].exec);
    if (g->pev) {
        for (int i = 0; i < g->n_pev; i++)
            if (g->pev[i]) qgpu_event_destroy(g->pev[i]);
        free(g->pev);
    }
    for (size_t i = 0; i < g->n_tensors; i++) qgpu_tensor_free(g->tensors[i]);
    for (size_t i = 0; i < g->n_allocs; i++) qgpu_free(g->allocs[i]);
    qgpu_host_free(g->h_acc);
    free(g->tensors);
    free(g->allocs);
    free(g->L);
    free(g);
}

/* ------------------------------------------------------------------ tensor sources */
typedef struct {
    const qwen_synth_spec_t *spec;    /* NULL: tensor bytes are t->data (mmap of a GGUF file) */
} source_t;

static const void *tensor_bytes(const source_t *src, const gguf_tensor_info_t *t, void **owned)
{
    *owned = NULL;
    if (!src->spec) return t->data;
    qwen_synth_tensor_t d;
    if (qwen_synth_describe(src->spec, (uint32_t)t->offset, &d)) return NULL;
    void *buf = malloc(d.nbytes ? d.nbytes : 1);
    if (!buf || qwen_synth_fill(src->spec, (uint32_t)t->offset, buf)) { free(buf); return NULL; }
    *owned = buf;
    return buf;
}

static qgpu_tensor *up_matrix(qwen_gpu_t *g, const source_t *src, const gguf_tensor_info_t *t)
{
    void *own;
    const void *bytes = tensor_bytes(src, t, &own);
    if (!bytes) return NULL;
    qgpu_tensor *T = NULL;
    int rc = qgpu_tensor_upload(bytes, (int)t->type, t->ne[0], t->n_dims >= 2 ? t->ne[1] : 1, &T);
    free(own);
    if (rc) { fprintf(stderr, "model_init: upload of %s failed: %s\n", t->name, qgpu_strerror(rc)); return NULL; }
    if (g->n_tensors == g->cap_tensors) {
        g->cap_tensors = g->cap_tensors ? 2 * g->cap_tensors : 256;
        g->tensors = realloc(g->tensors, g->cap_tensors * sizeof(qgpu_tensor *));
    }
    g->tensors[g->n_tensors++] = T;
    return T;
}

static float *up_f32(qwen_gpu_t *g, const source_t *src, const gguf_tensor_info_t *t)
{
    if (t->type != GGML_F32) { fprintf(stderr, "model_init: %s must be F32\n", t->name); return NULL; }
    const size_t n = (size_t)t->ne[0] * (t->n_dims >= 2 ? t->ne[1] : 1);
    void *own;
    const void *bytes = tensor_bytes(src, t, &own);
    float *d = bytes ? dalloc(g, n * sizeof(float)) : NULL;
    if (d && qgpu_memcpy_h2d(d, bytes, n * sizeof(float))) d = NULL;
    free(own);
    return d;
}

/* ------------------------------------------------------------------ binding (model.c:31-147,239-284) */
static const gguf_tensor_info_t *need(const gguf_context_t *g, const char *name)
{
    const gguf_tensor_info_t *t = gguf_find_tensor(g, name);
    if (!t) fprintf(stderr, "model_init: missing tensor %s\n", name);
    return t;
}
static int bad2(const gguf_tensor_info_t *t, uint64_t a, uint64_t b, const char *what)
{
    if (!t) return 1;
    if (t->n_dims != 2 || t->ne[0] != a || t->ne[1] != b) { fprintf(stderr, "model_init: %s dimension mismatch\n", what); return 1; }
    return 0;
}
static int bad1(const gguf_tensor_info_t *t, uint64_t a, const char *what)
{
    if (!t) return 1;
    if (t->n_dims != 1 || t->ne[0] != a) { fprintf(stderr, "model_init: %s dimension mismatch\n", what); return 1; }
    return 0;
}

static int bind_layer(const gguf_context_t *G, qwen_layer_t *L, uint32_t il, const qwen_dims_t *d, int mtp)
{
    char nm[96];
#define B_(field, fmt) do { snprintf(nm, sizeof nm, fmt, il); if (!(L->field = need(G, nm))) return -1; } while (0)
    B_(attn_norm, "blk.%u.attn_norm.weight");
    B_(post_attn_norm, "blk.%u.post_attention_norm.weight");
    B_(ffn_gate, "blk.%u.ffn_gate.weight");
    B_(ffn_up, "blk.%u.ffn_up.weight");
    B_(ffn_down, "blk.%u.ffn_down.weight");
    if (bad2(L->ffn_gate, d->n_embd, d->n_ff, "ffn_gate") || bad2(L->ffn_up, d->n_embd, d->n_ff, "ffn_up") ||
        bad2(L->ffn_down, d->n_ff, d->n_embd, "ffn_down") || bad1(L->attn_norm, d->n_embd, "attn_norm") ||
        bad1(L->post_attn_norm, d->n_embd, "post_attention_norm"))
        return -1;
    if (L->is_recurrent) {
        B_(wqkv, "blk.%u.attn_qkv.weight"); B_(wqkv_gate, "blk.%u.attn_gate.weight");
        B_(ssm_conv1d, "blk.%u.ssm_conv1d.weight"); B_(ssm_dt_bias, "blk.%u.ssm_dt.bias");
        B_(ssm_a, "blk.%u.ssm_a"); B_(ssm_beta, "blk.%u.ssm_beta.weight");
        B_(ssm_alpha, "blk.%u.ssm_alpha.weight"); B_(ssm_norm, "blk.%u.ssm_norm.weight");
        B_(ssm_out, "blk.%u.ssm_out.weight");
        if (bad2(L->wqkv, d->n_embd, d->conv_dim, "wqkv") || bad2(L->wqkv_gate, d->n_embd, d->d_inner, "wqkv_gate") ||
            bad2(L->ssm_conv1d, d->d_conv, d->conv_dim, "ssm_conv1d") ||
            bad2(L->ssm_beta, d->n_embd, d->n_v_heads, "ssm_beta") ||
            bad2(L->ssm_alpha, d->n_embd, d->n_v_heads, "ssm_alpha") ||
            bad2(L->ssm_out, d->d_inner, d->n_embd, "ssm_out") || bad1(L->ssm_dt_bias, d->n_v_heads, "ssm_dt_bias") ||
            bad1(L->ssm_a, d->n_v_heads, "ssm_a") || bad1(L->ssm_norm, d->head_v_dim, "ssm_norm"))
            return -1;
    } else {
        B_(attn_q, "blk.%u.attn_q.weight"); B_(attn_k, "blk.%u.attn_k.weight"); B_(attn_v, "blk.%u.attn_v.weight");
        B_(attn_q_norm, "blk.%u.attn_q_norm.weight"); B_(attn_k_norm, "blk.%u.attn_k_norm.weight");
        B_(attn_out, "blk.%u.attn_output.weight");
        if (bad2(L->attn_q, d->n_embd, 2 * d->n_head * d->head_dim, "attn_q") ||
            bad2(L->attn_k, d->n_embd, d->n_kv_head * d->head_dim, "attn_k") ||
            bad2(L->attn_v, d->n_embd, d->n_kv_head * d->head_dim, "attn_v") ||
            bad2(L->attn_out, d->n_head * d->head_dim, d->n_embd, "attn_out") ||
            bad1(L->attn_q_norm, d->head_dim, "attn_q_norm") || bad1(L->attn_k_norm, d->head_dim, "attn_k_norm"))
            return -1;
    }
#undef B_
    (void)mtp;
    return 0;
}

static int upload_layer(qwen_gpu_t *g, const source_t *src, const qwen_layer_t *L, glayer_t *D)
{
    D->rec = L->is_recurrent;
    if (!(D->attn_norm = up_f32(g, src, L->attn_norm)) || !(D->post_norm = up_f32(g, src, L->post_attn_norm)) ||
        !(D->ffn_gate = up_matrix(g, src, L->ffn_gate)) || !(D->ffn_up = up_matrix(g, src, L->ffn_up)) ||
        !(D->ffn_down = up_matrix(g, src, L->ffn_down)))
        return -1;
    if (L->is_recurrent) {
        if (!(D->wqkv = up_matrix(g, src, L->wqkv)) || !(D->wgate = up_matrix(g, src, L->wqkv_gate)) ||
            !(D->beta = up_matrix(g, src, L->ssm_beta)) || !(D->alpha = up_matrix(g, src, L->ssm_alpha)) ||
            !(D->ssm_out = up_matrix(g, src, L->ssm_out)) || !(D->conv1d = up_f32(g, src, L->ssm_conv1d)) ||
            !(D->dt_bias = up_f32(g, src, L->ssm_dt_bias)) || !(D->ssm_a = up_f32(g, src, L->ssm_a)) ||
            !(D->ssm_norm = up_f32(g, src, L->ssm_norm)))
            return -1;
    } else {
        if (!(D->q = up_matrix(g, src, L->attn_q)) || !(D->k = up_matrix(g, src, L->attn_k)) ||
            !(D->v = up_matrix(g, src, L->attn_v)) || !(D->o = up_matrix(g, src, L->attn_out)) ||
            !(D->q_norm = up_f32(g, src, L->attn_q_norm)) || !(D->k_norm = up_f32(g, src, L->attn_k_norm)))
            return -1;
    }
    return 0;
}

static int model_load(qwen_model_t *m, const source_t *src, uint32_t n_ctx)
{
    qwen_config_t *c = &m->cfg;
    qwen_dims_t *d = &m->dims;
    *c = m->gguf.config;
    d->n_embd = c->n_embd; d->n_ff = c->n_ff; d->n_head = c->n_head; d->n_kv_head = c->n_head_kv;
    d->head_dim = c->head_dim; d->n_k_heads = c->ssm_group_count; d->head_k_dim = d->head_v_dim = c->ssm_state_size;
    d->d_inner = c->ssm_inner_size; d->d_conv = c->ssm_conv_kernel; d->d_state = c->ssm_state_size;
    memcpy(d->rope_sections, c->rope_sections, sizeof d->rope_sections);
    const gguf_tensor_info_t *a0 = gguf_find_tensor(&m->gguf, "blk.0.ssm_a");
    if (!a0 || a0->n_dims != 1) { fprintf(stderr, "model_init: blk.0.ssm_a missing\n"); return -1; }
    d->n_v_heads = (uint32_t)a0->ne[0];
    d->conv_dim = 2 * d->n_k_heads * d->head_k_dim + d->d_inner;
    d->n_layer = c->n_layer > c->nextn_layers ? c->n_layer - c->nextn_layers : c->n_layer;
    if (d->d_inner != d->n_v_heads * d->head_v_dim || d->n_v_heads > 256 || d->head_v_dim > 256 ||
        d->head_k_dim > 256 || !c->full_attn_interval) {
        fprintf(stderr, "model_init: inconsistent GDN dimensions\n");
        return -1;
    }
    /* shapes the GPU kernels are written for */
    if (d->head_k_dim != 128 || d->head_dim != 256 || d->d_conv != 4 || c->rope_dim_count > d->head_dim ||
        d->n_embd % 256 || d->n_ff % 256 || !d->n_kv_head || d->n_head % d->n_kv_head ||
        (d->n_head / d->n_kv_head) * MAXB > 48 || d->d_inner > d->n_ff) {
        fprintf(stderr, "model_init: dimensions outside what the GPU kernels support\n");
        return -1;
    }
    m->tok_embd = need(&m->gguf, "token_embd.weight");
    m->output_norm = need(&m->gguf, "output_norm.weight");
    m->output = gguf_find_tensor(&m->gguf, "output.weight");
    if (!m->output) m->output = m->tok_embd;
    if (!m->tok_embd || !m->output_norm || bad2(m->tok_embd, d->n_embd, c->vocab_size, "token_embd")) return -1;
    m->layers = calloc(d->n_layer, sizeof *m->layers);
    if (!m->layers) return -1;
    for (uint32_t il = 0; il < d->n_layer; il++) {
        m->layers[il].is_recurrent = ((il + 1) % c->full_attn_interval) != 0;
        if (bind_layer(&m->gguf, &m->layers[il], il, d, 0)) return -1;
        if (m->layers[il].is_recurrent) d->n_recr_layer++;
        else d->n_attn_layer++;
    }
    {
        qwen_layer_t *L = &m->mtp_layer;
        memset(L, 0, sizeof *L);
        const uint32_t il = d->n_layer;
        if (bind_layer(&m->gguf, L, il, d, 1)) return -1;
        char nm[96];
        snprintf(nm, sizeof nm, "blk.%u.nextn.eh_proj.weight", il);
        m->mtp_eh_proj = need(&m->gguf, nm);
        snprintf(nm, sizeof nm, "blk.%u.nextn.enorm.weight", il);
        m->mtp_enorm = need(&m->gguf, nm);
        snprintf(nm, sizeof nm, "blk.%u.nextn.hnorm.weight", il);
        m->mtp_hnorm = need(&m->gguf, nm);
        snprintf(nm, sizeof nm, "blk.%u.nextn.shared_head_norm.weight", il);
        m->mtp_shnorm = need(&m->gguf, nm);
        if (bad2(m->mtp_eh_proj, 2 * d->n_embd, d->n_embd, "nextn.eh_proj") || bad1(m->mtp_enorm, d->n_embd, "nextn.enorm") ||
            bad1(m->mtp_hnorm, d->n_embd, "nextn.hnorm") || bad1(m->mtp_shnorm, d->n_embd, "nextn.shared_head_norm"))
            return -1;
    }
    if (n_ctx < 2) { fprintf(stderr, "model_init: n_ctx must be at least 2\n"); return -1; }
    if (n_ctx > 0x7FFFFFFFu || !qgpu_attn_cache_fits((int)n_ctx, (int)d->n_kv_head)) {
        fprintf(stderr, "model_init: n_ctx %u: a KV cache of %u heads is beyond what the attention kernels address "
                "(%u x %u x 1 KiB > 2 GiB)\n", n_ctx, d->n_kv_head, n_ctx, d->n_kv_head);
        return -1;
    }
    m->n_ctx = n_ctx;
    m->pos = 0;

    if (qwen_dev_err) { fprintf(stderr, "model_init: an earlier device error is pending\n"); return -1; }
    if (qgpu_init(0)) { fprintf(stderr, "model_init: no GPU\n"); return -1; }
    qwen_gpu_t *g = calloc(1, sizeof *g);
    m->gpu = g;
    {
        /* QWEN_GRAPHS=1: replay captured launch sequences.  Measured on MI355X the
         * 27B verify step is the same either way (the per-kernel cost is inside the
         * kernels, not the dispatch), so kernels are launched from the host by default. */
        const char *ge = getenv("QWEN_GRAPHS");
        g->use_graphs = ge && ge[0] == '1';
        const char *pe = getenv("QWEN_PROFILE");
        g->prof = pe && pe[0] && pe[0] != '0';
        /* QWEN_GDN_FACTOR_MIN_B=n: forwards of n tokens or more keep the GDN state in factor form
         * (default 5; 9 turns it off).  Measured on MI355X at the 27B shapes: a GDN layer at B = 8
         * writes one state instead of 8 snapshots, at B <= 4 the snapshots cost about the same. */
        const char *fe = getenv("QWEN_GDN_FACTOR_MIN_B");
        g->factor_min_b = fe && atoi(fe) >= 1 ? atoi(fe) : 5;
        g->fbase = -1;
    }
    g->L = calloc(d->n_layer, sizeof *g->L);
    for (uint32_t il = 0; il < d->n_layer; il++)
        if (upload_layer(g, src, &m->layers[il], &g->L[il])) return -1;
    if (upload_layer(g, src, &m->mtp_layer, &g->mtp)) return -1;
    if (!(g->tok_embd = up_matrix(g, src, m->tok_embd))) return -1;
    {   /* the first preparation of a forward gathers the embedding rows itself (packed IQ4_XS) */
        int t;
        uint64_t ne0, ne1;
        const char *ef = getenv("QWEN_EMBD_FUSE");   /* "0": a separate dequant launch, as for other formats */
        g->embd_fuse = !(ef && ef[0] == '0') && !qgpu_tensor_shape(g->tok_embd, &t, &ne0, &ne1) &&
                       t == GGML_IQ4_XS && ne0 % 256 == 0 && ne0 <= 64 * 256;
    }
    g->output = (m->output == m->tok_embd) ? g->tok_embd : up_matrix(g, src, m->output);
    if (!g->output || !(g->eh_proj = up_matrix(g, src, m->mtp_eh_proj)) ||
        !(g->out_norm = up_f32(g, src, m->output_norm)) || !(g->enorm = up_f32(g, src, m->mtp_enorm)) ||
        !(g->hnorm = up_f32(g, src, m->mtp_hnorm)) || !(g->shnorm = up_f32(g, src, m->mtp_shnorm)))
        return -1;

    const uint64_t E = d->n_embd, F = d->n_ff, V = c->vocab_size;
    g->kvrow = (uint64_t)d->n_kv_head * d->head_dim;
    g->conv_elems = (uint64_t)d->conv_dim * 4;
    g->ssm_elems = (uint64_t)d->n_v_heads * d->head_v_dim * d->head_k_dim;
    g->f_tok = ((uint64_t)(d->n_v_heads + d->n_k_heads) * d->head_v_dim + d->n_v_heads + 3) & ~3ull;
    uint64_t SQ = d->conv_dim;
    if (2ull * d->n_head * d->head_dim > SQ) SQ = 2ull * d->n_head * d->head_dim;
    if (F > SQ) SQ = F;
    if (2 * E > SQ) SQ = 2 * E;
    g->SQ = (SQ + 3) & ~3ull;
    g->A = (uint64_t)d->n_head * d->head_dim > d->d_inner ? (uint64_t)d->n_head * d->head_dim : d->d_inner;
    const size_t kvb = (size_t)n_ctx * g->kvrow * sizeof(float);
    for (uint32_t il = 0; il <= d->n_layer; il++) {
        glayer_t *D = il < d->n_layer ? &g->L[il] : &g->mtp;
        if (D->rec) {
            D->conv_ring = dalloc(g, NSLOT * g->conv_elems * sizeof(float));
            D->ssm_ring = dalloc(g, NSLOT * g->ssm_elems * sizeof(float));
            D->gdn_f = dalloc(g, 2 * MAXB * g->f_tok * sizeof(float));
            if (!D->conv_ring || !D->ssm_ring || !D->gdn_f) return -1;
        } else {
            D->kv_k = dalloc(g, kvb);
            D->kv_v = dalloc(g, kvb);
            if (!D->kv_k || !D->kv_v) return -1;
        }
    }
#define AL(p, n) do { if (!((p) = dalloc(g, (n) * sizeof(*(p))))) return -1; } while (0)
    AL(g->d_fst, 2); AL(g->d_fstv, 2 * 2 * NSLOT);
    AL(g->d_pos, 4); AL(g->d_cur, 4); AL(g->d_posv, (uint64_t)n_ctx + MAXB); AL(g->d_curv, NSLOT); AL(g->d_tok, 64); AL(g->d_cand, 64); AL(g->d_vtok, 64); AL(g->d_acc, 64);
    AL(g->anchor_tok, 64); AL(g->anchor_h, E);
    if (qgpu_host_malloc((void **)&g->h_acc, 64 * sizeof(uint32_t))) return -1;
    AL(g->bx, MAXB * E); AL(g->bxb, MAXB * E); AL(g->bqkv, MAXB * g->SQ); AL(g->bk, MAXB * g->kvrow);
    AL(g->bv, MAXB * g->kvrow); AL(g->bz, MAXB * (uint64_t)d->d_inner);
    /* gate inputs: up to QGPU_MAX_KS partial planes of MAXB rows (gdn_dev) */
    AL(g->bbeta, QGPU_MAX_KS * MAXB * (uint64_t)d->n_v_heads + 4);
    AL(g->balpha, QGPU_MAX_KS * MAXB * (uint64_t)d->n_v_heads + 4);
    AL(g->bffn, MAXB * F); AL(g->battn, MAXB * g->A); AL(g->xq, MAXB * (uint64_t)d->conv_dim);
    AL(g->h_save, MAXB * E); AL(g->logits_b, MAXB * V); AL(g->logits1, V); AL(g->mtp_h, E);
    AL(g->mx, MAXB * E); AL(g->cat, MAXB * 2 * E); AL(g->part, 8 * MAXB * E);
#undef AL
    {   /* position and ring-slot tables: entry i holds i */
        const uint64_t np = (uint64_t)n_ctx + MAXB;
        int *tab = malloc(np * sizeof(int));
        if (!tab) return -1;
        for (uint64_t i = 0; i < np; i++) tab[i] = (int)i;
        const int bad = qgpu_memcpy_h2d(g->d_posv, tab, np * sizeof(int)) ||
                        qgpu_memcpy_h2d(g->d_curv, tab, NSLOT * sizeof(int));
        free(tab);
        if (bad) return -1;
        int fst[2 * 2 * NSLOT];                 /* entry 2 * P + par: {P, par} */
        for (int i = 0; i < 2 * NSLOT; i++) { fst[2 * i] = i >> 1; fst[2 * i + 1] = i & 1; }
        if (qgpu_memcpy_h2d(g->d_fstv, fst, sizeof fst)) return -1;
    }
    g->fst_ptr = g->d_fst;
    g->pos_ptr = g->d_pos;
    g->cur_ptr = g->d_cur;
    /* RoPE tables with the reference's own expressions (model.c:186-201) */
    const uint32_t half = c->rope_dim_count / 2;
    float *cs = malloc((size_t)n_ctx * half * sizeof(float)), *sn = malloc((size_t)n_ctx * half * sizeof(float));
    if (!cs || !sn) { free(cs); free(sn); return -1; }
    for (uint32_t p = 0; p < n_ctx; p++)
        for (uint32_t i = 0; i < half; i++) {
            const float angle = (float)p * powf(c->rope_theta, -2.0f * (float)i / (float)c->rope_dim_count);
            cs[(size_t)p * half + i] = cosf(angle);
            sn[(size_t)p * half + i] = sinf(angle);
        }
    g->rope_cos = dalloc(g, (size_t)n_ctx * half * sizeof(float));
    g->rope_sin = dalloc(g, (size_t)n_ctx * half * sizeof(float));
    int rc = (!g->rope_cos || !g->rope_sin) ? -1 :
             (qgpu_memcpy_h2d(g->rope_cos, cs, (size_t)n_ctx * half * sizeof(float)) ||
              qgpu_memcpy_h2d(g->rope_sin, sn, (size_t)n_ctx * half * sizeof(float)));
    m->rope_cos = cs;                          /* host copies (reference field names) */
    m->rope_sin = sn;
    if (rc || qgpu_attn_reserve((int)n_ctx, (int)d->n_kv_head)) return -1;
    for (int b = 1; b <= QGPU_MAX_B; b++)
        g->att_split[b] = qgpu_attn_split_bound((int)n_ctx, b, (int)d->n_head, (int)d->n_kv_head);
    /* host-side fields, laid out as the reference's arenas (model.c:166-230) */
    {
        const uint64_t sq = g->SQ > F ? g->SQ : F, kvs = 2ull * d->n_kv_head * d->head_dim;
        const uint64_t hd = (uint64_t)d->n_head * d->head_dim;
        float *p = m->arena = calloc(2 * E + sq + kvs + d->d_inner + F + hd + V + (uint64_t)d->n_head * n_ctx,
                                     sizeof(float));
        if (!p) return -1;
        m->x = p; p += E;
        m->xb = p; p += E;
        m->qkv = p; p += sq;
        m->kv_small = p; p += kvs;
        m->z = p; p += d->d_inner;
        m->ffn_buf = p; p += F;
        m->attn_out = p; p += hd;
        m->logits = p; p += V;
        m->scores = p;
        p = m->arena_b = calloc(MAXB * (2 * E + F + kvs + d->d_inner + F + hd + E), sizeof(float));
        if (!p) return -1;
        m->bx = p; p += MAXB * E;
        m->bxb = p; p += MAXB * E;
        m->bqkv = p; p += MAXB * F;
        m->bkv = p; p += MAXB * kvs;
        m->bz = p; p += MAXB * (uint64_t)d->d_inner;
        m->bffn = p; p += MAXB * F;
        m->battn_out = p; p += MAXB * hd;
        m->h_save = p;
        m->logits_b = calloc(MAXB * V, sizeof(float));
        m->mtp_h = calloc(E, sizeof(float));
        if (!m->logits_b || !m->mtp_h) return -1;
    }
    m->host_sync = 1;
    g->cur = g->cur_base = 0;
    if (qgpu_sync()) return -1;
    return 0;
}

int model_init(qwen_model_t *m, const char *path, uint32_t n_ctx)
{
    memset(m, 0, sizeof *m);
    if (gguf_open(&m->gguf, path) != 0) return -1;
    source_t src = { NULL };
    if (model_load(m, &src, n_ctx)) { model_free(m); return -1; }
    return 0;
}

/* a generated tensor table stands in for the GGUF file: offset = synth index */
int model_init_synth(qwen_model_t *m, const qwen_synth_spec_t *s, uint32_t n_ctx)
{
    memset(m, 0, sizeof *m);
    m->gguf.fd = -1;
    m->gguf.alignment = 32;
    snprintf(m->gguf.arch, sizeof m->gguf.arch, "qwen35");
    const uint32_t nt = qwen_synth_count(s);
    m->gguf.tensors = calloc(nt, sizeof(gguf_tensor_info_t));
    m->gguf.tensor_count = nt;
    m->gguf.header.tensor_count = nt;
    for (uint32_t i = 0; i < nt; i++) {
        qwen_synth_tensor_t d;
        qwen_synth_describe(s, i, &d);
        gguf_tensor_info_t *t = &m->gguf.tensors[i];
        memcpy(t->name, d.name, GGUF_MAX_NAME);
        t->n_dims = d.n_dims;
        t->ne[0] = d.ne[0];
        t->ne[1] = d.n_dims >= 2 ? d.ne[1] : 1;
        t->ne[2] = t->ne[3] = 1;
        t->type = (ggml_type_t)d.type;
        t->offset = i;
        t->data = NULL;
    }
    qwen_config_t *c = &m->gguf.config;
    c->n_embd = s->n_embd; c->n_head = s->n_head; c->n_head_kv = s->n_kv_head; c->head_dim = s->head_dim;
    c->n_layer = s->n_layer + 1; c->n_ff = s->n_ff; c->vocab_size = s->vocab; c->context_len = s->context_len;
    c->rope_theta = s->rope_theta; c->rope_dim_count = s->rope_dim;
    c->rope_sections[0] = 11; c->rope_sections[1] = 11; c->rope_sections[2] = 10; c->rope_sections[3] = 0;
    c->rms_norm_eps = s->eps; c->full_attn_interval = s->full_attn_interval; c->ssm_state_size = s->state;
    c->ssm_conv_kernel = 4; c->ssm_inner_size = s->n_v_heads * s->state; c->ssm_group_count = s->n_k_heads;
    c->nextn_layers = 1;
    source_t src = { s };
    if (model_load(m, &src, n_ctx)) { model_free(m); return -1; }
    return 0;
}

void model_free(qwen_model_t *m)
{
    if (!m) return;
    gpu_free(m->gpu);
    free(m->layers);
    free(m->arena); free(m->arena_b); free(m->logits_b); free(m->mtp_h); free(m->rope_cos); free(m->rope_sin);
    if (m->gguf.fd >= 0 || m->gguf.mmap_data) gguf_close(&m->gguf);
    else free(m->gguf.tensors);
    memset(m, 0, sizeof *m);
}

/* ------------------------------------------------------------------ device layers */
/* activation transforms fused into the GEMV input preparation (include/qgpu.h) */
static qgpu_act act_norm(const float *x, uint64_t ldx, const float *w, float eps, float *xout, uint64_t ldxo)
{
    qgpu_act a;
    memset(&a, 0, sizeof a);
    a.kind = QGPU_ACT_RMSNORM; a.x = x; a.ldx = ldx; a.w = w; a.eps = eps; a.xout = xout; a.ldxo = ldxo;
    return a;
}

/* adds the pending partial planes into their residual (in place) */
static void materialize(qwen_model_t *m)
{
    qwen_gpu_t *g = m->gpu;
    const uint64_t E = m->dims.n_embd;
    if (g->pend_tok) {
        K(qgpu_dequant_rows(g->tok_embd, g->pend_tok, (int)g->pend_tok_B, g->bx, E));
        g->pend_tok = NULL;
    }
    if (!g->pend_ks) return;
    K(qgpu_add_partials(g->pend, E, g->pend, E, g->part, E, g->pend_ks, E, (int)g->pend_B));
    g->pend_ks = 0;
    g->pend = NULL;
}

/* RMSNorm of residual R as a GEMV input; pending partial planes of R are added
 * in (and written back to R) by the same preparation kernel */
static qgpu_act act_norm_res(qwen_model_t *m, float *R, const float *w, float *xout)
{
    qwen_gpu_t *g = m->gpu;
    const uint64_t E = m->dims.n_embd;
    if ((g->pend_ks && g->pend != R) || (g->pend_tok && R != g->bx)) materialize(m);
    qgpu_act a = act_norm(R, E, w, m->cfg.rms_norm_eps, xout, E);
    if (g->pend_tok) {   /* the embedding rows: gathered by this preparation, which writes them to R */
        a.x = NULL; a.embd = g->tok_embd; a.tok = g->pend_tok; a.xnew = R; a.ldxn = E;
        g->pend_tok = NULL;
    }
    if (g->pend_ks) {
        a.part = g->part; a.ldp = E; a.n_part = g->pend_ks; a.xnew = R; a.ldxn = E;
        g->pend_ks = 0;
        g->pend = NULL;
    }
    return a;
}

/* R += W v (reference residual adds, model.c:466,483,942): narrow matrices run
 * K-split and leave their partial planes pending on R */
static void residual_gemv(qwen_model_t *m, const qgpu_tensor *W, const qgpu_act *act, uint32_t B, float *R)
{
    qwen_gpu_t *g = m->gpu;
    const uint64_t E = m->dims.n_embd;
    materialize(m);
    const int ks = qgpu_gemv_split_ks(W);
    if (ks > 1) {
        K(qgpu_gemv_act_split(W, act, (int)B, g->part, E, ks));
        g->pend = R; g->pend_ks = ks; g->pend_B = B;
    } else {
        K(qgpu_gemv_act_batch(&W, 1, act, (int)B, &R, &E, QGPU_GEMV_ACCUM));
    }
}

/* residual_gemv on the input the previous kernel prepared (packed matrices only) */
static void residual_gemv_prepared(qwen_model_t *m, const qgpu_tensor *W, uint32_t B, float *R)
{
    qwen_gpu_t *g = m->gpu;
    const uint64_t E = m->dims.n_embd;
    materialize(m);
    const int ks = qgpu_gemv_split_ks(W);
    if (ks > 1) {
        K(qgpu_gemv_prepared_split(W, (int)B, g->part, E, ks));
        g->pend = R; g->pend_ks = ks; g->pend_B = B;
    } else {
        K(qgpu_gemv_prepared(W, (int)B, R, E, QGPU_GEMV_ACCUM));
    }
}

/* matrices that run on the matrix cores (packed tile records): the formats with
 * an MFMA kernel and whole 256-column super-blocks */
static int mat_packed(const qgpu_tensor *W)
{
    int t;
    uint64_t ne0, ne1;
    if (qgpu_tensor_shape(W, &t, &ne0, &ne1)) return 0;
    return (t == GGML_IQ4_XS || t == GGML_Q4_K || t == GGML_Q5_K || t == GGML_Q6_K ||
            t == GGML_Q8_0) && ne0 % 256 == 0;
}

/* where a preparation writes its fp32 rows: only when a matrix it feeds runs on the VALU kernel,
 * which reads them (the matrix-core GEMV reads the digit planes) */
static float *rows_for(const qgpu_tensor *const *W, int n, float *buf)
{
    for (int i = 0; i < n; i++)
        if (!mat_packed(W[i])) return buf;
    return NULL;
}

static void ffn_dev(qwen_model_t *m, glayer_t *D, float *R, uint32_t B)
{
    qwen_gpu_t *g = m->gpu;
    const uint64_t F = m->dims.n_ff;
    /* post-attention RMSNorm -> gate/up (model.c:469-476) */
    const qgpu_tensor *W[2] = { D->ffn_gate, D->ffn_up };
    const qgpu_act an = act_norm_res(m, R, D->post_norm, rows_for(W, 2, g->bxb));
    float *outs[2] = { g->bffn, g->bqkv };
    const uint64_t ld[2] = { F, g->SQ };
    K(qgpu_gemv_act_batch(W, 2, &an, (int)B, outs, ld, 0));
    /* silu(gate) * up -> down, residual add (model.c:477-483) */
    qgpu_act sm;
    memset(&sm, 0, sizeof sm);
    sm.kind = QGPU_ACT_SILU_MUL; sm.x = g->bffn; sm.ldx = F; sm.y = g->bqkv; sm.ldy = g->SQ;
    if (rows_for((const qgpu_tensor *const *)&D->ffn_down, 1, g->bffn)) { sm.xout = g->bffn; sm.ldxo = F; }
    residual_gemv(m, D->ffn_down, &sm, B, R);
}

static void attn_dev(qwen_model_t *m, glayer_t *D, float *R, uint32_t B, uint32_t pos)
{
    qwen_gpu_t *g = m->gpu;
    const qwen_dims_t *d = &m->dims;
    const float eps = m->cfg.rms_norm_eps;
    const qgpu_tensor *W[3] = { D->q, D->k, D->v };
    const qgpu_act an = act_norm_res(m, R, D->attn_norm, rows_for(W, 3, g->bxb));
    float *outs[3] = { g->bqkv, g->bk, g->bv };
    const uint64_t ld[3] = { g->SQ, g->kvrow, g->kvrow };
    K(qgpu_gemv_act_batch(W, 3, &an, (int)B, outs, ld, 0));
    /* q/k norm + RoPE + cache write + attention in one kernel, then the span merge, which also
     * prepares the o-projection input when the matrix runs on the matrix cores */
    (void)pos;   /* positions come from g->pos_ptr (at()); the grid covers n_ctx (spans past the live end exit) */
    const int prep = mat_packed(D->o);
    if (prep)
        K(qgpu_attn_fused_act_live(g->bqkv, g->SQ, g->bk, g->bv, g->kvrow, D->q_norm, D->k_norm, D->kv_k, D->kv_v,
                                   g->rope_cos, g->rope_sin, (int)m->cfg.rope_dim_count, g->pos_ptr, (int)m->n_ctx,
                                   (int)B, (int)d->n_head, (int)d->n_kv_head, (int)d->head_dim, eps, NULL, g->A,
                                   g->att_live));        /* digit planes only: the o-projection reads them */
    else
        K(qgpu_attn_fused(g->bqkv, g->SQ, g->bk, g->bv, g->kvrow, D->q_norm, D->k_norm, D->kv_k, D->kv_v,
                          g->rope_cos, g->rope_sin, (int)m->cfg.rope_dim_count, g->pos_ptr, (int)m->n_ctx, (int)B,
                          (int)d->n_head, (int)d->n_kv_head, (int)d->head_dim, eps, g->battn, g->A));
    if (prep) {
        residual_gemv_prepared(m, D->o, B, R);
    } else {
        qgpu_act oc;
        memset(&oc, 0, sizeof oc);
        oc.kind = QGPU_ACT_COPY; oc.x = g->battn; oc.ldx = g->A;
        residual_gemv(m, D->o, &oc, B, R);
    }
    ffn_dev(m, D, R, B);
}

static void gdn_dev(qwen_model_t *m, glayer_t *D, uint32_t B)
{
    qwen_gpu_t *g = m->gpu;
    const qwen_dims_t *d = &m->dims;
    const uint64_t di = d->d_inner;
    const float eps = m->cfg.rms_norm_eps;
    const qgpu_tensor *W[4] = { D->wqkv, D->wgate, D->beta, D->alpha };
    const qgpu_act an = act_norm_res(m, g->bx, D->attn_norm, rows_for(W, 4, g->bxb));
    float *outs[4] = { g->bqkv, g->bz, g->bbeta, g->balpha };
    const uint64_t ld[4] = { g->SQ, di, d->n_v_heads, d->n_v_heads };
    /* beta and alpha (n_v_heads rows each: a few tiles) are cut into one K range per 256-column
     * super-block, so their bytes spread over many compute units instead of adding a whole tile to a
     * few (with 1024 + 6 tiles, 6 compute units would stream 5 tiles and the rest 4); the GDN kernel
     * sums the partial planes */
    int kba = 1;
    if (mat_packed(D->beta) && mat_packed(D->alpha)) {
        kba = (int)(d->n_embd / 256);
        if (kba > QGPU_MAX_KS) kba = QGPU_MAX_KS;
        if (kba * (int)B > 256) kba = 256 / (int)B;
    }
    const int ks[4] = { 1, 1, kba, kba };
    K(qgpu_gemv_act_batch_ks(W, 4, &an, (int)B, outs, ld, ks));
    /* conv1d + SiLU + L2 norms + delta rule over the B tokens, state snapshots into the ring */
    K(qgpu_gdn_fused_factor(g->bqkv, g->SQ, (int)B, (int)d->conv_dim, D->conv1d, D->conv_ring, g->conv_elems,
                            g->bbeta, g->balpha, d->n_v_heads, kba, (uint64_t)B * d->n_v_heads, D->dt_bias,
                            D->ssm_a, D->ssm_ring, g->ssm_elems, NSLOT, g->cur_ptr, (int)d->n_k_heads,
                            (int)d->n_v_heads, (int)d->head_v_dim, eps, g->battn, di, D->gdn_f, g->f_tok,
                            g->fst_ptr, (int)B >= g->factor_min_b));
    /* per-head gated RMSNorm (model.c:928-941) fused into the ssm_out input */
    qgpu_act gn;
    memset(&gn, 0, sizeof gn);
    gn.kind = QGPU_ACT_GATED_NORM; gn.x = g->battn; gn.ldx = di; gn.y = g->bz; gn.ldy = di; gn.w = D->ssm_norm;
    gn.seg = d->head_v_dim; gn.eps = eps;
    if (rows_for((const qgpu_tensor *const *)&D->ssm_out, 1, g->bffn)) { gn.xout = g->bffn; gn.ldxo = di; }
    residual_gemv(m, D->ssm_out, &gn, B, g->bx);
    ffn_dev(m, D, g->bx, B);
}

/* Section timing of model_forward (reference model.c:697-742, printed by main.c
 * --profile): while prof_active, forward_body records an event before the
 * embedding, after it, after every layer and after the head; prof_collect then
 * adds the device time between consecutive events to qwen_prof_embed,
 * qwen_prof_gdn / qwen_prof_attn (by layer kind) and qwen_prof_head.  It is on
 * when QWEN_PROFILE is set in the environment at model_init (the reference's
 * compile-time switch of that name) or after qwen_model_set_profile(m, 1). */
static void prof_mark(qwen_gpu_t *g, uint32_t i)
{
    if (g->prof_active) K(qgpu_event_record(g->pev[i]));
}

static int prof_begin(qwen_model_t *m)
{
    qwen_gpu_t *g = m->gpu;
    if (!g->prof || qwen_dev_err) return 0;
    if (!g->pev) {
        g->pev = calloc(m->dims.n_layer + 3, sizeof *g->pev);
        if (!g->pev) return 0;
        g->n_pev = (int)m->dims.n_layer + 3;
        for (uint32_t i = 0; i < m->dims.n_layer + 3; i++) K(qgpu_event_create(&g->pev[i]));
        if (qwen_dev_err) return 0;
    }
    g->prof_active = 1;
    return 1;
}

static void prof_collect(qwen_model_t *m)
{
    qwen_gpu_t *g = m->gpu;
    const uint32_t nl = m->dims.n_layer;
    g->prof_active = 0;
    for (uint32_t i = 0; i <= nl + 1 && !qwen_dev_err; i++) {
        float ms = 0.0f;
        K(qgpu_event_elapsed_ms(g->pev[i], g->pev[i + 1], &ms));
        const double sec = 1e-3 * (double)ms;
        if (i == 0) qwen_prof_embed += sec;
        else if (i == nl + 1) qwen_prof_head += sec;
        else if (g->L[i - 1].rec) qwen_prof_gdn += sec;
        else qwen_prof_attn += sec;
    }
}

/* Graph cache: the launch sequence of a body depends only on its pointers, B
 * and flag (positions and the GDN ring index are read from device memory), so
 * it is captured once and replayed; replay cuts the per-kernel launch gap. */
enum { G_FWD = 1, G_MTP = 2 };
typedef void (*body_fn)(qwen_model_t *, const uint32_t *, const float *, uint32_t, float *, int);

static void run_body(qwen_model_t *m, int kind, body_fn fn, const uint32_t *tok, const float *h, uint32_t B,
                     float *lg, int flag)
{
    qwen_gpu_t *g = m->gpu;
    if (!g->use_graphs || g->prof_active) { fn(m, tok, h, B, lg, flag); return; }
    for (int i = 0; i < g->n_graphs; i++)
        if (g->graphs[i].kind == kind && g->graphs[i].tok == tok && g->graphs[i].h == h && g->graphs[i].lg == lg &&
            g->graphs[i].B == B && g->graphs[i].flag == flag && g->graphs[i].live == g->att_live) {
            K(qgpu_graph_launch(g->graphs[i].exec));
            return;
        }
    if (g->n_graphs == (int)(sizeof g->graphs / sizeof g->graphs[0])) { fn(m, tok, h, B, lg, flag); return; }
    void *exec = NULL;
    K(qgpu_graph_begin());
    fn(m, tok, h, B, lg, flag);
    K(qgpu_graph_end(&exec));
    const int i = g->n_graphs++;
    g->graphs[i].kind = kind; g->graphs[i].tok = tok; g->graphs[i].h = h; g->graphs[i].lg = lg;
    g->graphs[i].B = B; g->graphs[i].flag = flag; g->graphs[i].live = g->att_live; g->graphs[i].exec = exec;
    K(qgpu_graph_launch(exec));
}

static void forward_body(qwen_model_t *m, const uint32_t *d_tokens, const float *unused, uint32_t B,
                         float *d_logits, int save_h)
{
    (void)unused;
    qwen_gpu_t *g = m->gpu;
    const qwen_dims_t *d = &m->dims;
    const uint64_t E = d->n_embd, V = m->cfg.vocab_size;
    prof_mark(g, 0);
    /* the first preparation gathers the rows itself; a profiled forward keeps the lookup a launch of
     * its own, so the embedding section times it (the two are bit-identical) */
    if (g->embd_fuse && !g->prof_active) { g->pend_tok = d_tokens; g->pend_tok_B = B; }
    else K(qgpu_dequant_rows(g->tok_embd, d_tokens, (int)B, g->bx, E));
    prof_mark(g, 1);
    for (uint32_t il = 0; il < d->n_layer; il++) {
        if (g->L[il].rec) gdn_dev(m, &g->L[il], B);
        else attn_dev(m, &g->L[il], g->bx, B, 0);
        prof_mark(g, 2 + il);
    }
    qgpu_act an = act_norm_res(m, g->bx, g->out_norm, rows_for((const qgpu_tensor *const *)&g->output, 1, g->bxb));
    /* when the last residual add is still pending (partial planes), its preparation writes the
     * final hidden states straight into h_save; bx then lacks those planes, and nothing reads
     * it before the next forward's embedding overwrites it */
    const int direct = save_h && an.n_part;
    if (direct) an.xnew = g->h_save;
    K(qgpu_gemv_act_batch((const qgpu_tensor *const *)&g->output, 1, &an, (int)B, &d_logits, &V, 0));
    prof_mark(g, 2 + d->n_layer);
    if (save_h && !direct) K(qgpu_copy(g->h_save, g->bx, B * E * sizeof(float)));
}

/* Where the kernels of the next launch sequence read the position and the ring slot.
 * Eager launches read the constant tables at the host's values (d_posv + pos, d_curv +
 * cur), so no kernel sets them; a captured graph reads d_pos / d_cur, which are set
 * before each replay (with_cur: the sequence has GDN layers). */
static int gdn_pending(const qwen_gpu_t *g)
{
    return g->fbase >= 0 ? (g->cur - g->fbase + NSLOT) % NSLOT : 0;
}

static void at(qwen_model_t *m, uint32_t pos, int with_cur);

/* Writes the state the ring index selects into slot cur of every GDN layer when it is still kept
 * as a base state plus factors (after a factor-form forward), so that nothing is pending.  The
 * other states of that forward are then gone: model_rollback_to is refused until the next forward. */
static void gdn_settle(qwen_model_t *m)
{
    qwen_gpu_t *g = m->gpu;
    if (!gdn_pending(g)) return;
    at(m, m->pos, 1);
    for (uint32_t il = 0; il < m->dims.n_layer; il++)
        if (g->L[il].rec)
            K(qgpu_gdn_materialize(g->L[il].ssm_ring, g->ssm_elems, NSLOT, g->cur_ptr, (int)m->dims.n_k_heads,
                                   (int)m->dims.n_v_heads, (int)m->dims.head_v_dim, g->L[il].gdn_f, g->f_tok,
                                   g->fst_ptr));
    g->fbase = -1;
    g->last_B = 0;
}

static void at(qwen_model_t *m, uint32_t pos, int with_cur)
{
    qwen_gpu_t *g = m->gpu;
    const int P = gdn_pending(g);
    if (g->use_graphs && !g->prof_active) {
        K(qgpu_set_i32(g->d_pos, (int)pos));
        if (with_cur) {
            K(qgpu_set_i32(g->d_cur, g->cur));
            K(qgpu_set_i32(g->d_fst, P));
            K(qgpu_set_i32(g->d_fst + 1, g->fpar));
        }
        g->pos_ptr = g->d_pos;
        g->cur_ptr = g->d_cur;
        g->fst_ptr = g->d_fst;
    } else {
        g->pos_ptr = g->d_posv + pos;
        g->cur_ptr = g->d_curv + g->cur;
        g->fst_ptr = g->d_fstv + 2 * (2 * P + g->fpar);
    }
}

/* tokens on the device; logits of every token into d_logits ([B][V]); hidden
 * states into h_save when save_h.  GDN states advance by B (ring index). */
/* the attention launches' live-context bound for B tokens at position pos */
static void att_bound(qwen_gpu_t *g, uint32_t pos, uint32_t B)
{
    const int b = B <= QGPU_MAX_B ? g->att_split[B] : 0;
    g->att_live = b && pos + B <= (uint32_t)b ? b : 0;
}

static void forward_dev(qwen_model_t *m, const uint32_t *d_tokens, uint32_t B, uint32_t pos, float *d_logits,
                        int save_h)
{
    qwen_gpu_t *g = m->gpu;
    at(m, pos, 1);
    att_bound(g, pos, B);
    run_body(m, G_FWD, forward_body, d_tokens, NULL, B, d_logits, save_h);
    if ((int)B >= g->factor_min_b) {              /* GDN state kept in slot cur, factors in the other buffer */
        g->fbase = g->cur;
        g->fpar ^= 1;
    } else {
        g->fbase = -1;
    }
    g->cur_base = g->cur;
    g->cur = (g->cur + (int)B) % NSLOT;
    g->last_B = (int)B;
}

static void mtp_body(qwen_model_t *m, const uint32_t *d_tokens, const float *h, uint32_t B, float *d_logits,
                     int unused);

/* MTP layer for B tokens (d_tokens) paired with hidden states h (device, [B][E]);
 * output rows in mx, mtp_h = last row; logits of every row into d_logits if given */
static void mtp_dev(qwen_model_t *m, const uint32_t *d_tokens, const float *h, uint32_t B, uint32_t pos,
                    float *d_logits)
{
    at(m, pos, 0);
    att_bound(m->gpu, pos, B);
    run_body(m, G_MTP, mtp_body, d_tokens, h, B, d_logits, 0);
}

/* MTP re-anchor of the speculative loop (main.c:219-221) on the token, hidden state and
 * position the acceptance kernel left on the device (anchor_tok, anchor_h, d_pos), so it
 * is enqueued before the host knows j; no logits */
static void mtp_anchor_dev(qwen_model_t *m)
{
    qwen_gpu_t *g = m->gpu;
    g->pos_ptr = g->d_pos;
    g->att_live = 0;              /* the position is the device's (no host bound) */
    run_body(m, G_MTP, mtp_body, g->anchor_tok, g->anchor_h, 1, NULL, 0);
}

static void mtp_body(qwen_model_t *m, const uint32_t *d_tokens, const float *h, uint32_t B, float *d_logits,
                     int unused)
{
    (void)unused;
    qwen_gpu_t *g = m->gpu;
    const uint64_t E = m->dims.n_embd, V = m->cfg.vocab_size;
    const float eps = m->cfg.rms_norm_eps;
    /* eh_proj(concat(enorm(e), hnorm(h))) (model.c:1044-1052): both norms in the input preparation,
     * which also gathers the embedding rows when it can */
    if (!g->embd_fuse) K(qgpu_dequant_rows(g->tok_embd, d_tokens, (int)B, g->bxb, E));
    /* with eh_proj on the matrix cores, no fp32 copy of the normalised input: the preparation then
     * leaves both row factors to the GEMV (one launch with per-element work only) */
    qgpu_act cat = act_norm(g->bxb, E, g->enorm, eps, mat_packed(g->eh_proj) ? NULL : g->cat, 2 * E);
    cat.y = h; cat.ldy = E; cat.w2 = g->hnorm; cat.seg = E;
    if (g->embd_fuse) { cat.x = NULL; cat.embd = g->tok_embd; cat.tok = d_tokens; }
    K(qgpu_gemv_act_batch((const qgpu_tensor *const *)&g->eh_proj, 1, &cat, (int)B, &g->mx, &E, 0));
    attn_dev(m, &g->mtp, g->mx, B, 0);
    /* mtp_h = the last output row.  With one row and the residual's partial planes still pending,
     * the kernel that adds them writes the row straight into mtp_h (mx then lacks them; nothing
     * reads mx before the next eh_proj overwrites it) */
    int direct = 0;
    if (d_logits) {
        qgpu_act an = act_norm_res(m, g->mx, g->shnorm, rows_for((const qgpu_tensor *const *)&g->output, 1, g->bxb));
        if (B == 1 && an.n_part) { an.xnew = g->mtp_h; direct = 1; }
        K(qgpu_gemv_act_batch((const qgpu_tensor *const *)&g->output, 1, &an, (int)B, &d_logits, &V, 0));
    } else if (B == 1 && g->pend_ks && g->pend == g->mx && g->pend_B == 1 && !g->pend_tok) {
        K(qgpu_add_partials(g->mtp_h, E, g->mx, E, g->part, E, g->pend_ks, E, 1));
        g->pend_ks = 0;
        g->pend = NULL;
        direct = 1;
    } else {
        materialize(m);
    }
    if (!direct) K(qgpu_copy(g->mtp_h, g->mx + (B - 1) * E, E * sizeof(float)));
}

/* ------------------------------------------------------------------ reference API */
static int bad_tokens(const qwen_model_t *m, const uint32_t *tokens, uint32_t B)
{
    for (uint32_t b = 0; b < B; b++)
        if (tokens[b] >= m->cfg.vocab_size) return 1;
    return 0;
}

static void put_tokens(qwen_model_t *m, const uint32_t *tokens, uint32_t B)
{
    K(qgpu_memcpy_h2d(m->gpu->d_tok, tokens, B * sizeof(uint32_t)));
}

void model_forward(qwen_model_t *m, pool_t *pool, uint32_t token, uint32_t pos)
{
    (void)pool;
    if (call_begin(m)) return;
    if (bad_span(m, pos, 1) || token >= m->cfg.vocab_size) { reject(m, "model_forward", pos, 1); return; }
    put_tokens(m, &token, 1);
    const int prof = prof_begin(m);
    forward_dev(m, m->gpu->d_tok, 1, pos, m->gpu->logits1, 0);
    if (prof) prof_collect(m);
    if (m->host_sync) {
        K(qgpu_memcpy_d2h(m->logits, m->gpu->logits1, (size_t)m->cfg.vocab_size * sizeof(float)));
        K(qgpu_memcpy_d2h(m->x, m->gpu->bx, m->dims.n_embd * sizeof(float)));
    }
    qwen_prof_calls++;
    m->pos = pos + 1;
    call_end(m);
}

void model_forward_batch(qwen_model_t *m, pool_t *pool, const uint32_t *tokens, uint32_t pos, uint32_t B, int ckpt)
{
    (void)pool;
    (void)ckpt;
    if (call_begin(m)) return;
    if (!tokens || bad_span(m, pos, B) || bad_tokens(m, tokens, B)) { reject(m, "model_forward_batch", pos, B); return; }
    put_tokens(m, tokens, B);
    forward_dev(m, m->gpu->d_tok, B, pos, m->gpu->logits_b, 1);
    if (m->host_sync) {
        K(qgpu_memcpy_d2h(m->logits_b, m->gpu->logits_b, (size_t)B * m->cfg.vocab_size * sizeof(float)));
        K(qgpu_memcpy_d2h(m->h_save, m->gpu->h_save, (size_t)B * m->dims.n_embd * sizeof(float)));
    }
    m->pos = pos + B;
    call_end(m);
}

void model_reset(qwen_model_t *m)
{
    if (call_begin(m)) return;
    qwen_gpu_t *g = m->gpu;
    for (uint32_t il = 0; il < m->dims.n_layer; il++) {
        const glayer_t *D = &g->L[il];
        if (!D->rec) continue;
        K(qgpu_memset(D->conv_ring, 0, NSLOT * g->conv_elems * sizeof(float)));
        K(qgpu_memset(D->ssm_ring, 0, NSLOT * g->ssm_elems * sizeof(float)));
    }
    g->cur = g->cur_base = 0;
    g->last_B = 0;
    g->fbase = -1;
    g->fpar = 0;
    g->pend_ks = 0;
    g->pend = NULL;
    K(qgpu_set_i32(g->d_cur, 0));
    K(qgpu_set_i32(g->d_pos, 0));
    K(qgpu_sync());
    m->pos = 0;
    call_end(m);
}

int model_snapshot_states(qwen_model_t *m) { (void)m; return 0; }
void model_rollback_states(qwen_model_t *m) { (void)m; }

void model_rollback_to(qwen_model_t *m, uint32_t b)
{
    if (call_begin(m)) return;
    qwen_gpu_t *g = m->gpu;
    /* the ring holds the states after tokens 0..B-1 of the last batch only */
    if (b >= SPEC_MAX_B || b >= (uint32_t)g->last_B) {
        fprintf(stderr, "model_rollback_to: state after token %u requested, the last batch had %d token(s); call ignored\n",
                b, g->last_B);
        g->status = -1;
        return;
    }
    g->cur = (g->cur_base + 1 + (int)b) % NSLOT;   /* the next forward reads it through at() */
    call_end(m);
}

int mtp_forward(qwen_model_t *m, pool_t *pool, uint32_t token, uint32_t pos, int want_logits)
{
    (void)pool;
    if (call_begin(m)) return -1;
    if (bad_span(m, pos, 1) || token >= m->cfg.vocab_size) return reject(m, "mtp_forward", pos, 1);
    qwen_gpu_t *g = m->gpu;
    const uint64_t E = m->dims.n_embd;
    if (m->host_sync) K(qgpu_memcpy_h2d(g->mtp_h, m->mtp_h, E * sizeof(float)));
    put_tokens(m, &token, 1);
    mtp_dev(m, g->d_tok, g->mtp_h, 1, pos, want_logits ? g->logits1 : NULL);
    if (m->host_sync) {
        K(qgpu_memcpy_d2h(m->mtp_h, g->mtp_h, E * sizeof(float)));
        if (want_logits) K(qgpu_memcpy_d2h(m->logits, g->logits1, (size_t)m->cfg.vocab_size * sizeof(float)));
    }
    call_end(m);
    return g->status;
}

int mtp_forward_batch(qwen_model_t *m, pool_t *pool, const uint32_t *tokens, uint32_t pos, uint32_t B,
                      int want_logits)
{
    (void)pool;
    if (call_begin(m)) return -1;
    if (!tokens || bad_span(m, pos, B) || bad_tokens(m, tokens, B)) return reject(m, "mtp_forward_batch", pos, B);
    qwen_gpu_t *g = m->gpu;
    put_tokens(m, tokens, B);
    mtp_dev(m, g->d_tok, g->h_save, B, pos, want_logits ? g->logits_b : NULL);
    if (m->host_sync) {
        K(qgpu_memcpy_d2h(m->mtp_h, g->mtp_h, m->dims.n_embd * sizeof(float)));
        if (want_logits)
            K(qgpu_memcpy_d2h(m->logits_b, g->logits_b, (size_t)B * m->cfg.vocab_size * sizeof(float)));
    }
    call_end(m);
    return g->status;
}

uint32_t model_sample_greedy(const float *logits, uint32_t vocab_size)
{
    uint32_t best = 0;
    float mv = logits[0];
    for (uint32_t i = 1; i < vocab_size; i++)
        if (logits[i] > mv) { mv = logits[i]; best = i; }
    return best;
}

void attention_layer(qwen_model_t *m, qwen_layer_t *L, pool_t *pool, uint32_t pos)
{
    (void)pool;
    if (call_begin(m)) return;
    if (bad_span(m, pos, 1) || !L || L->is_recurrent) { reject(m, "attention_layer", pos, 1); return; }
    qwen_gpu_t *g = m->gpu;
    glayer_t *D = (L == &m->mtp_layer) ? &g->mtp : &g->L[L - m->layers];
    K(qgpu_memcpy_h2d(g->bx, m->x, m->dims.n_embd * sizeof(float)));
    at(m, pos, 0);
    att_bound(g, pos, 1);
    attn_dev(m, D, g->bx, 1, pos);
    materialize(m);
    K(qgpu_memcpy_d2h(m->x, g->bx, m->dims.n_embd * sizeof(float)));
    call_end(m);
}

void gdn_layer(qwen_model_t *m, qwen_layer_t *L, pool_t *pool)
{
    (void)pool;
    if (call_begin(m)) return;
    if (!L || !L->is_recurrent || L < m->layers || L >= m->layers + m->dims.n_layer) {
        reject(m, "gdn_layer", 0, 1);
        return;
    }
    qwen_gpu_t *g = m->gpu;
    K(qgpu_memcpy_h2d(g->bx, m->x, m->dims.n_embd * sizeof(float)));
    glayer_t *D = &g->L[L - m->layers];
    gdn_settle(m);                        /* this call updates one layer in place: every state a snapshot first */
    at(m, m->pos, 1);
    gdn_dev(m, D, 1);
    materialize(m);
    /* the reference updates this layer's state in place (model.c:640-661): copy
     * the new state (slot cur+1) over the current slot so other layers keep theirs */
    const int nxt = (g->cur + 1) % NSLOT;
    K(qgpu_copy(D->conv_ring + (size_t)g->cur * g->conv_elems, D->conv_ring + (size_t)nxt * g->conv_elems,
                g->conv_elems * sizeof(float)));
    K(qgpu_copy(D->ssm_ring + (size_t)g->cur * g->ssm_elems, D->ssm_ring + (size_t)nxt * g->ssm_elems,
                g->ssm_elems * sizeof(float)));
    K(qgpu_memcpy_d2h(m->x, g->bx, m->dims.n_embd * sizeof(float)));
    call_end(m);
}

/* ------------------------------------------------------------------ device-resident generation */
/* returns the rows of the last chunk: the prompt's last logits row is logits_b[last - 1] */
static uint32_t prefill_dev(qwen_model_t *m, const uint32_t *prompt, uint32_t n, int with_mtp)
{
    qwen_gpu_t *g = m->gpu;
    uint32_t pos = 0, last = 0;
    while (pos < n) {
        const uint32_t B = n - pos > PREFILL_MAX_B ? PREFILL_MAX_B : n - pos;
        put_tokens(m, prompt + pos, B);
        forward_dev(m, g->d_tok, B, pos, g->logits_b, 1);
        if (with_mtp) mtp_dev(m, g->d_tok, g->h_save, B, pos, NULL);
        pos += B;
        last = B;
    }
    m->pos = n;
    /* next token = argmax of the last prompt row (main.c:148-151, 175) */
    K(qgpu_argmax(g->logits_b + (size_t)(last - 1) * m->cfg.vocab_size, m->cfg.vocab_size, m->cfg.vocab_size, 1,
                  g->d_cand));
    return last;
}

int model_spec_begin(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t k)
{
    if (call_begin(m)) return -1;
    if (!prompt || n_prompt < 1 || n_prompt >= m->n_ctx || bad_tokens(m, prompt, n_prompt))
        return reject(m, "model_spec_begin", 0, n_prompt);
    const uint32_t last = prefill_dev(m, prompt, n_prompt, k > 0);
    if (m->host_sync)             /* the last prompt row, where main.c:146-150 leaves it */
        K(qgpu_memcpy_d2h(m->logits, m->gpu->logits_b + (size_t)(last - 1) * m->cfg.vocab_size,
                          (size_t)m->cfg.vocab_size * sizeof(float)));
    K(qgpu_sync());
    call_end(m);
    return m->gpu->status;
}

#define ACC_PENDING 0xFFFFFFFFu

/* Waits for the acceptance kernel's result in pinned host memory: h_acc[0] leaves ACC_PENDING
 * once the rest is written.  After ~0.5 s of polling the stream is drained instead (a slow or
 * failed device; the error is recorded and the loop stops). */
static int wait_acc(qwen_model_t *m, uint32_t *acc, uint32_t n)
{
    qwen_gpu_t *g = m->gpu;
    if (qwen_dev_err) return -1;
    const double t0 = now_s();
    for (uint64_t spin = 1; __atomic_load_n(&g->h_acc[0], __ATOMIC_ACQUIRE) == ACC_PENDING; spin++)
        if (!(spin & 4095) && now_s() - t0 > 0.5) {
            K(qgpu_sync());
            if (qwen_dev_err) return -1;
            if (__atomic_load_n(&g->h_acc[0], __ATOMIC_ACQUIRE) == ACC_PENDING) { fail_rc("wait_acc", -1); return -1; }
            break;
        }
    for (uint32_t i = 0; i < n; i++) acc[i] = __atomic_load_n(&g->h_acc[i], __ATOMIC_ACQUIRE);
    return 0;
}

uint32_t model_spec_run(qwen_model_t *m, uint32_t k, uint32_t eos, int force_accept, uint32_t max_cycles,
                        uint32_t max_tokens, uint32_t *out, uint32_t *cycle_j, qwen_gen_stats_t *st)
{
    qwen_gen_stats_t s;
    memset(&s, 0, sizeof s);
    if (st) *st = s;
    if (call_begin(m)) return 0;
    if (!out && max_tokens) { reject(m, "model_spec_run", m->pos, 1); return 0; }
    qwen_gpu_t *g = m->gpu;
    const uint32_t V = m->cfg.vocab_size;
    const uint64_t E = m->dims.n_embd;
    if (k > SPEC_MAX_B - 1) k = SPEC_MAX_B - 1;
    const double t0 = now_s();
    uint32_t gen = 0, kk = 0, j = 0;
    uint32_t acc[24] = { 0 }, next0 = 0;
    K(qgpu_memcpy_d2h(&next0, g->d_cand, sizeof next0));          /* argmax of the last verified row */
    while (!qwen_dev_err && gen < max_tokens && s.n_cycles < max_cycles && m->pos >= 1 && m->pos < m->n_ctx) {
        const uint32_t P = m->pos - 1;
        const uint32_t room = m->n_ctx - 1 - P;                    /* >= 1: pos < n_ctx */
        kk = k < room - 1 ? k : room - 1;
        if (next0 == eos) break;                                   /* main.c:179 */
        /* drafts: cand[s] = argmax MTP(cand[s-1], P+s) (main.c:182-185) */
        for (uint32_t d = 1; d <= kk; d++) {
            mtp_dev(m, g->d_cand + (d - 1), g->mtp_h, 1, P + d, g->logits1);
            K(qgpu_argmax(g->logits1, V, V, 1, g->d_cand + d));
        }
        /* batched verification (main.c:189) and argmax of every row */
        forward_dev(m, g->d_cand, kk + 1, P + 1, g->logits_b, 1);
        K(qgpu_argmax(g->logits_b, V, V, (int)(kk + 1), g->d_vtok));
        /* acceptance + GDN rollback on the device (main.c:191-217) */
        const int force_j = force_accept == 1 ? (int)kk : force_accept == 2 ? (int)(s.n_cycles % (kk + 1)) : -1;
        /* the verify left the position at P+kk+2: the reference stops there once it reaches the
         * context end, before any rollback or re-anchor (main.c:210) */
        const int ctx_end = P + kk + 2 >= m->n_ctx, anchor = !ctx_end && k > 0;
        /* the result goes to pinned host memory, j (h_acc[0]) last; d_pos = P+j+1 (pos0 = P), the
         * re-anchor's position; the next cand[0] = argmax logits_b[j] goes to d_cand[0] */
        __atomic_store_n(&g->h_acc[0], ACC_PENDING, __ATOMIC_RELEASE);
        K(qgpu_spec_accept_anchor(g->d_cand, g->d_vtok, (int)kk, force_j, (int)P, g->cur_base, g->d_pos,
                                  g->d_cur, NSLOT, g->h_acc, g->h_save, E, (int)E, anchor ? g->anchor_h : NULL,
                                  anchor ? g->anchor_tok : NULL, ctx_end ? NULL : g->d_cand));
        /* the re-anchor (MTP on the backbone hidden state of the last accepted token, main.c:220-222)
         * is enqueued before the host waits for j */
        if (anchor) mtp_anchor_dev(m);
        if (wait_acc(m, acc, kk + 3)) break;
        j = acc[0] <= kk ? acc[0] : kk;
        g->cur = (g->cur_base + 1 + (int)j) % NSLOT;
        if (cycle_j) cycle_j[s.n_cycles] = j;
        for (uint32_t i = 0; i <= j && gen < max_tokens; i++) out[gen++] = acc[1 + i];
        s.n_accepted += j;
        s.n_drafts += kk;
        s.n_cycles++;
        if (ctx_end) { m->pos = P + kk + 2; break; }
        m->pos = P + j + 2;
        next0 = acc[j + 2];
    }
    K(qgpu_sync());
    if (m->host_sync && s.n_cycles) {
        /* the last verify's rows (row j starts the next cycle) and the MTP state */
        K(qgpu_memcpy_d2h(m->logits_b, g->logits_b, (size_t)(kk + 1) * V * sizeof(float)));
        K(qgpu_memcpy_d2h(m->h_save, g->h_save, (size_t)(kk + 1) * E * sizeof(float)));
        K(qgpu_memcpy_d2h(m->mtp_h, g->mtp_h, E * sizeof(float)));
    }
    s.t_decode_s = now_s() - t0;
    if (st) *st = s;
    call_end(m);
    return gen;
}

uint32_t model_generate_spec(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                             uint32_t k, uint32_t eos, int force_accept, uint32_t *out, uint32_t *cycle_j,
                             qwen_gen_stats_t *st)
{
    const double t0 = now_s();
    if (st) memset(st, 0, sizeof *st);
    if (model_spec_begin(m, prompt, n_prompt, k)) return 0;
    const double t_prefill = now_s() - t0;
    const uint32_t n = model_spec_run(m, k, eos, force_accept, UINT32_MAX, n_predict, out, cycle_j, st);
    if (st) st->t_prefill_s = t_prefill;
    return n;
}

uint32_t model_generate_greedy(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                               uint32_t eos, uint32_t *out, qwen_gen_stats_t *st)
{
    qwen_gen_stats_t s;
    memset(&s, 0, sizeof s);
    if (st) *st = s;
    if (call_begin(m)) return 0;
    if (!prompt || !out || n_prompt < 1 || n_prompt >= m->n_ctx || n_predict < 1 || bad_tokens(m, prompt, n_prompt)) {
        reject(m, "model_generate_greedy", 0, n_prompt);
        return 0;
    }
    qwen_gpu_t *g = m->gpu;
    const uint32_t V = m->cfg.vocab_size;
    double t0 = now_s();
    prefill_dev(m, prompt, n_prompt, 0);
    K(qgpu_sync());
    s.t_prefill_s = now_s() - t0;
    t0 = now_s();
    uint32_t gen = 0, cur = 0;
    K(qgpu_memcpy_d2h(&cur, g->d_cand, sizeof cur));
    out[gen++] = cur;
    while (!qwen_dev_err && gen < n_predict && cur != eos && m->pos < m->n_ctx) {
        forward_dev(m, g->d_cand, 1, m->pos, g->logits1, 0);
        K(qgpu_argmax(g->logits1, V, V, 1, g->d_cand));
        K(qgpu_memcpy_d2h(&cur, g->d_cand, sizeof cur));
        m->pos++;
        out[gen++] = cur;
        s.n_cycles++;
    }
    K(qgpu_sync());
    s.t_decode_s = now_s() - t0;
    if (st) *st = s;
    call_end(m);
    return gen;
}

uint32_t model_generate_sample(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                               float temp, float top_p, uint32_t top_k, float repeat_penalty, uint64_t seed,
                               uint32_t eos, uint32_t *out, qwen_gen_stats_t *st)
{
    qwen_gen_stats_t s;
    memset(&s, 0, sizeof s);
    if (st) *st = s;
    if (call_begin(m)) return 0;
    if (!prompt || !out || n_prompt < 1 || n_prompt >= m->n_ctx || n_predict < 1 || bad_tokens(m, prompt, n_prompt)) {
        reject(m, "model_generate_sample", 0, n_prompt);
        return 0;
    }
    qwen_gpu_t *g = m->gpu;
    const uint32_t V = m->cfg.vocab_size;
    /* the fields sampler_init sets (sampler.c:46-56) */
    if (!top_k) top_k = 40;
    if (repeat_penalty <= 0.0f) repeat_penalty = 1.0f;
    uint64_t rng = seed ? seed : 0x123456789abcdefULL;
    const uint32_t last_n = 64;
    /* all_tokens of main.c: the prompt, then every sampled token, on the device */
    uint32_t *d_all = NULL;
    uint64_t *d_rng = NULL;
    K(qgpu_malloc((void **)&d_all, ((size_t)n_prompt + n_predict) * sizeof(uint32_t)));
    K(qgpu_malloc((void **)&d_rng, sizeof(uint64_t)));
    K(qgpu_memcpy_h2d(d_all, prompt, (size_t)n_prompt * sizeof(uint32_t)));
    K(qgpu_memcpy_h2d(d_rng, &rng, sizeof rng));
    uint32_t n_all = n_prompt;
    double t0 = now_s();
    const uint32_t last = prefill_dev(m, prompt, n_prompt, 0);
    K(qgpu_sync());
    s.t_prefill_s = now_s() - t0;
    t0 = now_s();
    /* main.c:233-246: sample from the last logits, forward the token, sample again */
    float *lg = g->logits_b + (size_t)(last - 1) * V;
    uint32_t gen = 0, cur = 0;
    while (!qwen_dev_err) {
        K(qgpu_sample(lg, V, d_all, n_all, temp, top_p, top_k, repeat_penalty, last_n, d_rng, d_all + n_all));
        K(qgpu_memcpy_d2h(&cur, d_all + n_all, sizeof cur));
        n_all++;
        out[gen++] = cur;
        if (gen >= n_predict || cur == eos || m->pos >= m->n_ctx) break;
        forward_dev(m, d_all + n_all - 1, 1, m->pos, g->logits1, 0);
        m->pos++;
        lg = g->logits1;
        s.n_cycles++;
    }
    K(qgpu_sync());
    s.t_decode_s = now_s() - t0;
    K(qgpu_free(d_all));
    K(qgpu_free(d_rng));
    if (st) *st = s;
    call_end(m);
    return gen;
}

int model_time_steps(qwen_model_t *m, uint32_t B, int reps, float *ms_verify, float *ms_decode, float *ms_draft)
{
    if (call_begin(m)) return -1;
    if (bad_span(m, m->pos, B) || reps < 1 || !ms_verify || !ms_decode) return reject(m, "model_time_steps", m->pos, B);
    qwen_gpu_t *g = m->gpu;
    gdn_settle(m);                      /* every rep then starts from the same snapshot state */
    const int cur0 = g->cur, base0 = g->cur_base, lastB0 = g->last_B, fbase0 = g->fbase, fpar0 = g->fpar;
    const uint32_t pos = m->pos;
    void *e0, *e1;
    K(qgpu_event_create(&e0));
    K(qgpu_event_create(&e1));
    /* verify: B tokens at pos (states are restored to the ring index after each rep) */
    forward_dev(m, g->d_cand, B, pos, g->logits_b, 1);
    g->cur = cur0; g->cur_base = base0; g->last_B = lastB0; g->fbase = fbase0; g->fpar = fpar0;
    K(qgpu_event_record(e0));
    for (int r = 0; r < reps; r++) {
        forward_dev(m, g->d_cand, B, pos, g->logits_b, 1);
        K(qgpu_argmax(g->logits_b, m->cfg.vocab_size, m->cfg.vocab_size, (int)B, g->d_vtok));
        g->cur = cur0; g->cur_base = base0; g->last_B = lastB0; g->fbase = fbase0; g->fpar = fpar0;
    }
    K(qgpu_event_record(e1));
    K(qgpu_event_elapsed_ms(e0, e1, ms_verify));
    *ms_verify /= (float)reps;
    K(qgpu_event_record(e0));
    for (int r = 0; r < reps; r++) {
        forward_dev(m, g->d_cand, 1, pos, g->logits1, 0);
        K(qgpu_argmax(g->logits1, m->cfg.vocab_size, m->cfg.vocab_size, 1, g->d_vtok));
        g->cur = cur0; g->cur_base = base0; g->last_B = lastB0; g->fbase = fbase0; g->fpar = fpar0;
    }
    K(qgpu_event_record(e1));
    K(qgpu_event_elapsed_ms(e0, e1, ms_decode));
    *ms_decode /= (float)reps;
    if (ms_draft) {
        const size_t eb = m->dims.n_embd * sizeof(float);
        float *keep = malloc(eb);                                  /* mtp_h is restored afterwards */
        K(qgpu_memcpy_d2h(keep, g->mtp_h, eb));
        K(qgpu_event_record(e0));
        for (int r = 0; r < reps; r++) {
            mtp_dev(m, g->d_cand, g->mtp_h, 1, pos, g->logits1);
            K(qgpu_argmax(g->logits1, m->cfg.vocab_size, m->cfg.vocab_size, 1, g->d_vtok));
        }
        K(qgpu_event_record(e1));
        K(qgpu_event_elapsed_ms(e0, e1, ms_draft));
        *ms_draft /= (float)reps;
        K(qgpu_memcpy_h2d(g->mtp_h, keep, eb));
        free(keep);
    }
    K(qgpu_sync());
    qgpu_event_destroy(e0);
    qgpu_event_destroy(e1);
    g->last_B = lastB0;
    call_end(m);
    return m->gpu->status;
}

/* ------------------------------------------------------------------ FFI helpers */
qwen_model_t *qwen_model_alloc(void) { return calloc(1, sizeof(qwen_model_t)); }
void qwen_model_dealloc(qwen_model_t *m) { free(m); }
float *qwen_model_field(qwen_model_t *m, const char *name)
{
    if (!strcmp(name, "logits")) return m->logits;
    if (!strcmp(name, "logits_b")) return m->logits_b;
    if (!strcmp(name, "h_save")) return m->h_save;
    if (!strcmp(name, "mtp_h")) return m->mtp_h;
    if (!strcmp(name, "x")) return m->x;
    return NULL;
}
uint32_t qwen_model_get(const qwen_model_t *m, const char *name)
{
    if (!strcmp(name, "pos")) return m->pos;
    if (!strcmp(name, "vocab")) return m->cfg.vocab_size;
    if (!strcmp(name, "n_embd")) return m->dims.n_embd;
    if (!strcmp(name, "n_ctx")) return m->n_ctx;
    if (!strcmp(name, "n_layer")) return m->dims.n_layer;
    return 0;
}
void qwen_model_set_pos(qwen_model_t *m, uint32_t pos) { m->pos = pos; }
int qwen_model_status(const qwen_model_t *m) { return (m && m->gpu) ? m->gpu->status : -1; }
void qwen_model_set_host_sync(qwen_model_t *m, int on) { m->host_sync = on; }
void qwen_model_set_graphs(qwen_model_t *m, int on) { if (m && m->gpu) m->gpu->use_graphs = on ? 1 : 0; }
void qwen_model_set_profile(qwen_model_t *m, int on) { if (m && m->gpu) m->gpu->prof = on ? 1 : 0; }
