/*
 * qwen_synth.h -- deterministic random-init weights for the hybrid model and
 * for standalone GEMV workloads (no counterpart in the reference, which only
 * loads real checkpoints; real weights are not available to this build).
 *
 * Every byte is a pure function of (seed, tensor id, block index): a
 * splitmix64 counter stream, Irwin-Hall normals built from exact integer sums,
 * correctly rounded float->half.  The same seed yields the same bytes on any
 * host, so a GGUF written here and the tensors generated straight into GPU
 * memory are identical.
 */
#ifndef QWEN_SYNTH_H
#define QWEN_SYNTH_H

#include "gguf.h"
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint32_t n_embd, n_ff, n_layer;          /* n_layer = backbone layers (MTP layer extra) */
    uint32_t n_head, n_kv_head, head_dim;
    uint32_t n_k_heads, n_v_heads, state;    /* GDN: group_count, dt_rank, head_k = head_v */
    uint32_t vocab, rope_dim, full_attn_interval, context_len;
    float    rope_theta, eps;
    int32_t  type_default;                   /* ggml type of every 2-D weight ...         */
    int32_t  type_embd, type_output, type_qkv, type_eh_proj;   /* ... unless overridden (<0 = default) */
    float    gain_output;                    /* output-RMS gain of the lm_head            */
    uint64_t seed;
    /* structure knobs (all zero = plain random init) */
    float    gain_embd;                      /* token-embedding RMS gain (0 = 1)          */
    float    gain_resid;                     /* gain of ffn_down, ssm_out, attn_output (0 = 0.5) */
    int32_t  mtp_diag;                       /* 1: the token half of nextn.eh_proj is a scaled
                                                identity plus weak noise, the hidden half weak
                                                noise (IQ4_XS only)                      */
    float    norm_sigma;                     /* spread of the RMSNorm weights around 1 (0 = 0.1) */
    int32_t  tie_shift;                      /* 1: output.weight row v = token_embd row v-1 (mod
                                                vocab), so the greedy next token of t is t+1
                                                unless the layers outweigh the embedding  */
    int32_t  tokenizer;                      /* 1: the GGUF also carries a byte-level BPE
                                                vocabulary (tokenizer.ggml.model "gpt2",
                                                .tokens, .merges): ids 0..255 the byte
                                                symbols, then a few merged tokens, fillers,
                                                and <|endoftext|>, <|im_start|>, <|im_end|>
                                                as the last three ids (vocab >= 300)     */
    int32_t  tie_output;                     /* 1: no output.weight tensor, so the lm_head is
                                                token_embd (the loader's fallback, model.c:87-88);
                                                2: output.weight is an exact copy of token_embd.
                                                Either way output.weight is listed last, so the
                                                other tensors of the two files are the same */
} qwen_synth_spec_t;

/* The 27B hybrid: 48 GDN + 16 GQA layers + MTP, H=5120, F=17408, V=248320, all IQ4_XS. */
void qwen_synth_spec_27b(qwen_synth_spec_t *s, uint64_t seed);
/* Small hybrid of the same structure for parity tests (dims in the body).
 * variant 0: every 2-D weight IQ4_XS; 1: the real checkpoint's format mix;
 * 2: a model whose MTP drafts agree with the backbone most of the time
 *    (output rows = embedding rows shifted by one, identity-like eh_proj,
 *    embeddings a little weaker than the layers' sum), so greedy speculative
 *    decoding accepts anywhere from 0 to k drafts per cycle. */
void qwen_synth_spec_tiny(qwen_synth_spec_t *s, uint64_t seed, int variant);

typedef struct {
    char     name[GGUF_MAX_NAME];
    uint32_t n_dims;
    uint64_t ne[2];
    int32_t  type;
    uint64_t nbytes;
    float    mu, sigma;                      /* F32 tensors: value = mu + sigma*z          */
    int32_t  neg_abs;                        /* F32: value = -(mu + sigma*|z|)             */
} qwen_synth_tensor_t;

/* Number of tensors of the model and the i-th descriptor (canonical order). */
uint32_t qwen_synth_count(const qwen_synth_spec_t *s);
int      qwen_synth_describe(const qwen_synth_spec_t *s, uint32_t i, qwen_synth_tensor_t *out);
/* Bytes of tensor i (out must hold nbytes). */
int      qwen_synth_fill(const qwen_synth_spec_t *s, uint32_t i, void *out);
/* Writes the whole model as a GGUF v3 file readable by gguf_open/model_init. */
int      qwen_synth_write_gguf(const qwen_synth_spec_t *s, const char *path);

/* Standalone matrix: ne1 rows of ne0 elements in ggml format `type`, with the
 * IQ4_XS/K-quant super-block scale d ~ fp16(|N(0,1)| * sigma_d); `id` keys
 * the stream.  Threads: 0 = auto. */
int qwen_synth_matrix(int32_t type, uint64_t ne0, uint64_t ne1, uint64_t seed, uint64_t id,
                      float sigma_d, void *out, int n_threads);
/* fp32 values mu + sigma*z, z ~ Irwin-Hall(12) normal, keyed by (seed, id). */
void qwen_synth_normal(float *out, uint64_t n, uint64_t seed, uint64_t id, float mu, float sigma);

/* correctly rounded (nearest-even) float -> IEEE half, subnormals included */
uint16_t qwen_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif
#endif
