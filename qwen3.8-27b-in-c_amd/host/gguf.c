/*
 * gguf.c -- GGUF v2/v3 reader (mmap, zero copy) filling qwen_config_t from
 * "<arch>.*" keys.  Implements include/gguf.h; replaces the reference
 * gguf.c:84-317 with the same acceptance rules (magic, version 2..3,
 * tensor_count in 1..100000, n_dims <= 4, exact key types, vocab fallback
 * from token_embd), and checks that every tensor's bytes lie inside the file.
 */
#define _POSIX_C_SOURCE 200809L
#include "gguf.h"
#include "quant.h"
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

size_t gguf_type_size(gguf_type_t t)
{
    static const unsigned char sz[13] = { 1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8 };
    return (unsigned)t < 13 ? sz[t] : 0;
}

typedef struct { const uint8_t *p, *end; } rd_t;

static int take(rd_t *r, void *dst, size_t n)
{
    if ((size_t)(r->end - r->p) < n) return -1;
    if (dst) memcpy(dst, r->p, n);
    r->p += n;
    return 0;
}

static int take_str(rd_t *r, char *dst, size_t cap)
{
    uint64_t n;
    if (take(r, &n, 8) || n > (uint64_t)(r->end - r->p)) return -1;
    if (dst) {
        size_t k = n < cap - 1 ? (size_t)n : cap - 1;
        memcpy(dst, r->p, k);
        dst[k] = 0;
    }
    r->p += n;
    return 0;
}

static int skip_val(rd_t *r, uint32_t t, int depth)
{
    if (depth > 4) return -1;
    if (t == GGUF_TYPE_STRING) return take_str(r, NULL, 0);
    if (t == GGUF_TYPE_ARRAY) {
        uint32_t et;
        uint64_t n;
        if (take(r, &et, 4) || take(r, &n, 8) || et > GGUF_TYPE_FLOAT64) return -1;
        const size_t es = gguf_type_size((gguf_type_t)et);
        if (es) {                               /* fixed-size elements: one bounds check */
            if (n > (uint64_t)(r->end - r->p) / es) return -1;
            r->p += n * es;
            return 0;
        }
        for (uint64_t i = 0; i < n; i++) if (skip_val(r, et, depth + 1)) return -1;
        return 0;
    }
    if (t > GGUF_TYPE_FLOAT64) return -1;
    return take(r, NULL, gguf_type_size((gguf_type_t)t));
}

struct key_slot { const char *suffix; gguf_type_t type; size_t off; };
#define CFG(f) offsetof(qwen_config_t, f)
static const struct key_slot k_slots[] = {
    { "embedding_length", GGUF_TYPE_UINT32, CFG(n_embd) },
    { "attention.head_count", GGUF_TYPE_UINT32, CFG(n_head) },
    { "attention.head_count_kv", GGUF_TYPE_UINT32, CFG(n_head_kv) },
    { "attention.key_length", GGUF_TYPE_UINT32, CFG(head_dim) },
    { "block_count", GGUF_TYPE_UINT32, CFG(n_layer) },
    { "feed_forward_length", GGUF_TYPE_UINT32, CFG(n_ff) },
    { "vocab_size", GGUF_TYPE_UINT32, CFG(vocab_size) },
    { "context_length", GGUF_TYPE_UINT32, CFG(context_len) },
    { "rope.freq_base", GGUF_TYPE_FLOAT32, CFG(rope_theta) },
    { "rope.dimension_count", GGUF_TYPE_UINT32, CFG(rope_dim_count) },
    { "attention.layer_norm_rms_epsilon", GGUF_TYPE_FLOAT32, CFG(rms_norm_eps) },
    { "tie_word_embeddings", GGUF_TYPE_BOOL, CFG(tie_word_embeddings) },
    { "full_attention_interval", GGUF_TYPE_UINT32, CFG(full_attn_interval) },
    { "ssm.state_size", GGUF_TYPE_UINT32, CFG(ssm_state_size) },
    { "ssm.conv_kernel", GGUF_TYPE_UINT32, CFG(ssm_conv_kernel) },
    { "ssm.inner_size", GGUF_TYPE_UINT32, CFG(ssm_inner_size) },
    { "ssm.group_count", GGUF_TYPE_UINT32, CFG(ssm_group_count) },
    { "nextn_predict_layers", GGUF_TYPE_UINT32, CFG(nextn_layers) },
};

/* key "<arch>.<suffix>" ?  returns the suffix or NULL */
static const char *arch_suffix(const char *key, const char *arch)
{
    const size_t n = strlen(arch);
    return (n && !strncmp(key, arch, n) && key[n] == '.') ? key + n + 1 : NULL;
}

static int read_meta(gguf_context_t *g, rd_t *r, int pass)
{
    for (uint64_t i = 0; i < g->header.metadata_kv_count; i++) {
        char key[160];
        uint32_t t;
        if (take_str(r, key, sizeof key) || take(r, &t, 4) || t > GGUF_TYPE_FLOAT64) return -1;
        if (pass == 1) {
            if (t == GGUF_TYPE_STRING && !strcmp(key, "general.architecture")) {
                if (take_str(r, g->arch, sizeof g->arch)) return -1;
                continue;
            }
            if (t == GGUF_TYPE_UINT32 && !strcmp(key, "general.alignment")) {
                uint32_t a;
                if (take(r, &a, 4)) return -1;
                if (a) g->alignment = a;
                continue;
            }
            if (skip_val(r, t, 0)) return -1;
            continue;
        }
        const char *suf = arch_suffix(key, g->arch);
        if (suf && t == GGUF_TYPE_ARRAY && !strcmp(suf, "rope.dimension_sections")) {
            uint32_t et;
            uint64_t n;
            if (take(r, &et, 4) || take(r, &n, 8)) return -1;
            if (et != GGUF_TYPE_UINT32 && et != GGUF_TYPE_INT32) return -1;
            for (uint64_t k = 0; k < n; k++) {
                uint32_t v;
                if (take(r, &v, 4)) return -1;
                if (k < 4) g->config.rope_sections[k] = v;
            }
            continue;
        }
        int hit = 0;
        if (suf)
            for (size_t k = 0; k < sizeof k_slots / sizeof k_slots[0]; k++)
                if ((uint32_t)k_slots[k].type == t && !strcmp(suf, k_slots[k].suffix)) {
                    uint8_t *dst = (uint8_t *)&g->config + k_slots[k].off;
                    if (t == GGUF_TYPE_BOOL) {
                        uint8_t b;
                        if (take(r, &b, 1)) return -1;
                        *(bool *)dst = b != 0;
                    } else if (take(r, dst, 4)) {
                        return -1;
                    }
                    hit = 1;
                    break;
                }
        if (!hit && skip_val(r, t, 0)) return -1;
    }
    return 0;
}

void gguf_close(gguf_context_t *g)
{
    if (!g) return;
    if (g->mmap_data) munmap((void *)g->mmap_data, g->file_size);
    if (g->fd >= 0) close(g->fd);
    free(g->tensors);
    memset(g, 0, sizeof *g);
    g->fd = -1;
}

int gguf_open(gguf_context_t *g, const char *path)
{
    memset(g, 0, sizeof *g);
    g->fd = -1;
    g->alignment = GGUF_DEFAULT_ALIGNMENT;
    const char *why = "open failed";
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) goto fail;
    struct stat st;
    why = "file too small";
    if (fstat(g->fd, &st) || st.st_size < (off_t)sizeof(gguf_header_t)) goto fail;
    g->file_size = (size_t)st.st_size;
    why = "mmap failed";
    void *map = mmap(NULL, g->file_size, PROT_READ, MAP_SHARED, g->fd, 0);
    if (map == MAP_FAILED) goto fail;
    g->mmap_data = map;
    rd_t r = { (const uint8_t *)map, (const uint8_t *)map + g->file_size };
    why = "bad header";
    if (take(&r, &g->header, sizeof g->header) || g->header.magic != GGUF_MAGIC) goto fail;
    why = "unsupported version";
    if (g->header.version < 2 || g->header.version > 3) goto fail;
    const uint8_t *kv = r.p;
    why = "bad metadata";
    if (read_meta(g, &r, 1) || !g->arch[0]) goto fail;
    r.p = kv;
    if (read_meta(g, &r, 2)) goto fail;
    why = "bad tensor count";
    if (g->header.tensor_count == 0 || g->header.tensor_count > 100000) goto fail;
    g->tensor_count = g->header.tensor_count;
    g->tensors = calloc(g->tensor_count, sizeof *g->tensors);
    why = "bad tensor table";
    if (!g->tensors) goto fail;
    for (uint64_t i = 0; i < g->tensor_count; i++) {
        gguf_tensor_info_t *t = &g->tensors[i];
        uint32_t ty;
        if (take_str(&r, t->name, sizeof t->name) || take(&r, &t->n_dims, 4) || t->n_dims > 4) goto fail;
        for (uint32_t d = 0; d < t->n_dims; d++) if (take(&r, &t->ne[d], 8)) goto fail;
        if (take(&r, &ty, 4) || take(&r, &t->offset, 8)) goto fail;
        t->type = (ggml_type_t)ty;
    }
    const uint64_t at = (uint64_t)(r.p - (const uint8_t *)map);
    const uint64_t base = (at + g->alignment - 1) / g->alignment * g->alignment;
    why = "data section outside file";
    if (base >= g->file_size) goto fail;
    g->data_base = (const uint8_t *)map + base;
    const uint64_t avail = g->file_size - base;
    for (uint64_t i = 0; i < g->tensor_count; i++) {
        gguf_tensor_info_t *t = &g->tensors[i];
        if (t->offset >= avail) goto fail;
        /* the whole tensor must lie in the file (types without a known row size
         * are only checked for their start; nothing here can compute on them) */
        const uint64_t rb = quant_row_bytes(t->type, t->ne[0]);
        uint64_t rows = 1;
        for (uint32_t d = 1; d < t->n_dims; d++) {
            if (t->ne[d] && rows > UINT64_MAX / t->ne[d]) goto fail;
            rows *= t->ne[d];
        }
        if (rb && (rows > (avail - t->offset) / rb)) goto fail;
        t->data = (const uint8_t *)g->data_base + t->offset;
    }
    if (!g->config.vocab_size) {
        const gguf_tensor_info_t *e = gguf_find_tensor(g, "token_embd.weight");
        if (e && e->n_dims == 2) g->config.vocab_size = (uint32_t)e->ne[1];
    }
    return 0;
fail:
    fprintf(stderr, "gguf_open(%s): %s\n", path, why);
    gguf_close(g);
    return -1;
}

const gguf_tensor_info_t *gguf_find_tensor(const gguf_context_t *g, const char *name)
{
    for (uint64_t i = 0; i < g->tensor_count; i++)
        if (!strcmp(g->tensors[i].name, name)) return &g->tensors[i];
    return NULL;
}
