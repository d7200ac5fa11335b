/*
 * oracle.h -- CPU restatement of the reference engine's MTP speculative-decode
 * path (quant formats, batched dequant-GEMV, ops, Gated-DeltaNet, gated GQA
 * attention, MTP layer, rollback, greedy spec cycle).
 *
 * THIS IS TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may link or call it, and only as the checker.
 * The product path (the HIP library and its C host layer) never calls it.
 *
 * Every function restates the reference function named in its comment
 * (file:line relative to the reference checkout).  Wherever the reference
 * uses 8-lane AVX2 accumulation the restatement emulates the same lanes and
 * the same reduction tree with scalar fmaf(), so results are bit-identical to
 * the compiled reference (pinned by tests/test_oracle_*.py against fixtures
 * produced from the reference build in oracle/_ref).
 */
#ifndef QWEN_ORACLE_H
#define QWEN_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (same numbering as the GGUF format, reference gguf.h:37-61) */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13,
       OR_Q6_K = 14, OR_IQ4_XS = 23 };

/* ---------------- quant formats (reference quant.c) ---------------- */
float  or_fp16_to_f32(uint16_t h);                                /* quant.c:6-28    */
size_t or_block_bytes(int type);                                  /* quant.c:34-45   */
size_t or_block_elems(int type);                                  /* quant.c:48-59   */
size_t or_row_bytes(int type, uint64_t ne0);                      /* quant.c:61-65   */
int    or_dequant_row(int type, const void *data, uint64_t ne0, float *dst); /* quant.c:184-208 */

/* ---------------- GEMV (reference kernels.c) ----------------
 * out[t*ldo + r] = dot(row r of W, x[t*ldx ...]) for t < n, r in [r0, r1).
 * W is ne1 rows of or_row_bytes(type, ne0) bytes each.               */
void or_gemv_rows_batch(int type, const void *W, uint64_t ne0,
                        const float *x, uint64_t ldx, int n,
                        float *out, uint64_t ldo, uint64_t r0, uint64_t r1); /* kernels.c:570-599 */
/* all rows, optionally split over n_threads pthreads (bit-identical for any split) */
void or_gemv_batch(int type, const void *W, uint64_t ne0, uint64_t ne1,
                   const float *x, uint64_t ldx, int n,
                   float *out, uint64_t ldo, int n_threads);           /* kernels.c:640-648 */

/* ---------------- ops (reference kernels.c:741-939) ---------------- */
void or_rmsnorm(float *out, const float *x, const float *w, uint64_t n, float eps);
void or_l2norm(float *out, const float *x, uint64_t n, float eps);
void or_silu_inplace(float *x, uint64_t n);
void or_sigmoid_inplace(float *x, uint64_t n);
void or_softplus_inplace(float *x, uint64_t n);
void or_softmax_inplace(float *x, uint64_t n);
float or_exp8_lane(float x);        /* one lane of exp256_ps, kernels.c:807-822 */
uint32_t or_argmax(const float *logits, uint32_t n);                 /* model.c:746-756 */

/* ---------------- Gated DeltaNet block (reference model.c:494-615,845-925) ------------
 * Restates one GDN layer's conv1d + SiLU + L2norm + delta-rule recurrence over
 * T tokens for given projection outputs, writing per-token state snapshots.
 *   qkv_raw : [T][conv_dim]  (wqkv projection outputs, before conv)
 *   beta_raw, alpha_raw : [T][n_v]
 *   conv_state : [conv_dim][4] in/out ; ssm_state : [n_v][hv][hk] in/out
 *   conv_w : [conv_dim][4]; dt_bias, ssm_a : [n_v]
 *   out : [T][n_v*hv] (recurrence output o, before gated norm)
 *   snap_conv : [T][conv_dim*4] or NULL ; snap_ssm : [T][n_v*hv*hk] or NULL
 *     (state after token b, for every b < T)                                     */
void or_gdn_block(int T, int conv_dim, int n_k, int n_v, int hk, int hv, float eps,
                  const float *qkv_raw, const float *beta_raw, const float *alpha_raw,
                  const float *conv_w, const float *dt_bias, const float *ssm_a,
                  float *conv_state, float *ssm_state, float *out,
                  float *snap_conv, float *snap_ssm);

/* ---------------- GGUF reader (reference gguf.c) ---------------- */
typedef struct {
    char        name[64];
    uint32_t    n_dims;
    uint64_t    ne[4];
    int         type;
    uint64_t    offset;
    const void *data;
} or_tensor_t;

typedef struct {
    uint32_t n_embd, n_head, n_head_kv, head_dim, n_layer, n_ff, vocab_size, context_len;
    float    rope_theta;
    uint32_t rope_dim_count, rope_sections[4];
    float    rms_norm_eps;
    uint32_t full_attn_interval, ssm_state_size, ssm_conv_kernel, ssm_inner_size,
             ssm_group_count, nextn_layers;
} or_config_t;

typedef struct or_model or_model_t;   /* opaque */

/* ---------------- model (reference model.c) ---------------- */
/* Loads a GGUF file; k_max = largest draft count the caller will use
 * (checkpoint slots = k_max; the reference fixes k_max = SPEC_MAX_B-1 = 2). */
or_model_t *or_model_open(const char *path, uint32_t n_ctx, uint32_t k_max);  /* model.c:55-290 */
void        or_model_close(or_model_t *m);                                   /* model.c:292-316 */
const or_config_t *or_model_config(const or_model_t *m);
int   or_model_n_layer(const or_model_t *m);
int   or_model_n_embd(const or_model_t *m);
uint32_t or_model_vocab(const or_model_t *m);
uint32_t or_model_pos(const or_model_t *m);
void  or_model_set_pos(or_model_t *m, uint32_t pos);
float *or_model_logits(or_model_t *m);        /* [vocab]            */
float *or_model_logits_b(or_model_t *m);      /* [B][vocab]         */
float *or_model_h_save(or_model_t *m);        /* [B][n_embd]        */
float *or_model_mtp_h(or_model_t *m);         /* [n_embd]           */
float *or_model_x(or_model_t *m);             /* [n_embd] residual  */
/* raw recurrent state of GDN layer index ir (0..n_recr-1) */
float *or_model_ssm_state(or_model_t *m, int ir);
float *or_model_conv_state(or_model_t *m, int ir);
void  or_model_set_threads(or_model_t *m, int n_threads);

void or_model_forward(or_model_t *m, uint32_t token, uint32_t pos);          /* model.c:714-744  */
void or_model_forward_batch(or_model_t *m, const uint32_t *tokens, uint32_t pos,
                            uint32_t B, int ckpt);                           /* model.c:976-1002 */
void or_model_rollback_to(or_model_t *m, uint32_t b);                        /* model.c:1015-1031*/
int  or_mtp_forward(or_model_t *m, uint32_t token, uint32_t pos, int want_logits); /* model.c:1038-1063 */
int  or_mtp_forward_batch(or_model_t *m, const uint32_t *tokens, uint32_t pos,
                          uint32_t B, int want_logits);                      /* model.c:1069-1103 */

/* ---------------- driver (reference main.c) ---------------- */
typedef struct {
    uint64_t n_cycles, n_accepted, n_drafts;
} or_spec_stats_t;
/* Prefill (main.c:133-152) then greedy MTP speculative decode (main.c:158-231)
 * with k drafts per cycle; eos = UINT32_MAX for none.  Returns tokens emitted. */
uint32_t or_generate_spec(or_model_t *m, const uint32_t *prompt, uint32_t n_prompt,
                          uint32_t n_predict, uint32_t k, uint32_t eos,
                          uint32_t *out, or_spec_stats_t *st, uint32_t *cycle_j);
/* ---------------- sampler (reference sampler.c, main.c:232-248) ---------------- */
typedef struct {
    float    temp;
    float    top_p;
    uint32_t top_k;
    float    repeat_penalty;
    uint32_t repeat_last_n;
    uint64_t rng_state;
} or_sampler_t;                                                   /* sampler.h:7-14  */
void     or_sampler_init(or_sampler_t *s, float temp, float top_p, uint32_t top_k, float repeat_penalty,
                         uint64_t seed);                          /* sampler.c:46-56 */
uint32_t or_sampler_sample(or_sampler_t *s, float *logits, uint32_t vocab, const uint32_t *tokens,
                           size_t n_tokens);                      /* sampler.c:62-162 */

/* Prefill then plain greedy decode with model_forward (main.c:232-248 with temp<=0). */
uint32_t or_generate_greedy(or_model_t *m, const uint32_t *prompt, uint32_t n_prompt,
                            uint32_t n_predict, uint32_t eos, uint32_t *out);
/* Prefill then the sampled decode of main.c:232-248 (sampler s advances in place). */
uint32_t or_generate_sample(or_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                            uint32_t eos, or_sampler_t *s, uint32_t *out);

#ifdef __cplusplus
}
#endif
#endif
