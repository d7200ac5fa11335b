/*
 * model.h -- hybrid Qwen model runtime on one MI355X (48 Gated-DeltaNet +
 * 16 gated-GQA layers + one MTP draft layer).
 *
 * Drop-in for the reference interface include/model.h:1-154: same type
 * names, same public fields read and written by the reference driver
 * (logits, logits_b, h_save, mtp_h, x, pos, dims, cfg, gguf) and the same
 * functions with the same arguments and return values.  Weights, KV caches,
 * recurrent states and activations live in GPU memory (the thread pool
 * argument is accepted and ignored).  With host_sync = 1 (the default after
 * model_init) every call leaves its results in the host-side fields exactly
 * where the reference leaves them, so reference callers (main.c's spec loop,
 * the test programs) run unchanged; with host_sync = 0 results stay on the
 * device and model_generate_spec() runs the whole speculative cycle there.
 *
 * Differences from the reference, by design:
 *   - SPEC_MAX_B is 8 (drafts k <= 7); the reference caps k at 2.
 *   - Recurrent-state checkpoints are a ring of state slots on the device;
 *     model_rollback_to() moves the ring index (no copy).  Batches of 5..8
 *     tokens keep the recurrent state as the batch's starting state plus one
 *     rank-1 factor per token (one state write instead of B); the next forward
 *     applies the factors up to the selected token first (QWEN_GDN_FACTOR_MIN_B
 *     sets the batch size from which this form is used; 9 turns it off).
 *   - Calls whose positions run past n_ctx (pos + B > n_ctx) are rejected on
 *     the host with a message, before any device work; the reference writes
 *     past its KV arrays.  After a rejected call or a device error,
 *     qwen_model_status() returns nonzero (the reference API has no error
 *     channel on the compute path); a device error is sticky: every later call
 *     does nothing.
 */
#if !defined(QWEN_MODEL_H) && !defined(MODEL_H)   /* either header, whichever came first */
#define QWEN_MODEL_H
/* the reference header of the same name is superseded by this one when both
   are on the include path (reference drivers compiled against this library) */
#define MODEL_H

#include "gguf.h"
#include "qwen_synth.h"
#include "threadpool.h"
#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {            /* reference model.h:10-31 */
    uint32_t n_embd, n_ff, n_layer, n_attn_layer, n_recr_layer;
    uint32_t n_head, n_kv_head, head_dim, rope_sections[4];
    uint32_t n_v_heads, n_k_heads, head_k_dim, head_v_dim, d_inner, conv_dim, d_conv, d_state;
} qwen_dims_t;

typedef struct {            /* reference model.h:33-57 */
    bool is_recurrent;
    const gguf_tensor_info_t *attn_norm, *post_attn_norm, *ffn_gate, *ffn_up, *ffn_down;
    const gguf_tensor_info_t *attn_q, *attn_k, *attn_v, *attn_q_norm, *attn_k_norm, *attn_out;
    const gguf_tensor_info_t *wqkv, *wqkv_gate, *ssm_conv1d, *ssm_dt_bias, *ssm_a, *ssm_beta, *ssm_alpha,
                             *ssm_norm, *ssm_out;
    /* States (reference model.h:53-56).  Here the KV caches and recurrent states
     * live in GPU memory (a ring of state slots per GDN layer), so these host
     * pointers stay NULL. */
    float *kv_k, *kv_v;
    float *conv_state;
    float *ssm_state;
} qwen_layer_t;

typedef struct qwen_gpu qwen_gpu_t;   /* device-side state (host/model.c) */

/* Field order and names of reference model.h:59-111, then this build's own
 * fields.  The host buffers are laid out as the reference lays them out
 * (model.c:166-230): one activation arena x | xb | qkv | kv_small | z | ffn_buf |
 * attn_out | logits | scores and one batch arena bx | bxb | bqkv | bkv | bz |
 * bffn | battn_out | h_save.  The device path writes the result fields (mtp_h,
 * x, logits, logits_b, h_save) when host_sync is on; the other buffers are host
 * scratch that reference callers may use (test_kernels.c passes xb to gemv). */
typedef struct {
    gguf_context_t gguf;          /* file metadata / tensor table (synthetic models: generated table) */
    qwen_config_t  cfg;
    qwen_dims_t    dims;
    qwen_layer_t  *layers;
    const gguf_tensor_info_t *tok_embd, *output_norm, *output;

    float *mtp_h;      /* [n_embd]        MTP hidden (input of the next mtp_forward)  */

    float *x;          /* [n_embd]        residual after the last single-token pass   */
    float *xb;         /* [n_embd]        host scratch                                */
    float *qkv;        /* [max(conv_dim, 2*n_head*head_dim, n_ff)] host scratch       */
    float *kv_small;   /* [2*n_kv_head*head_dim] host scratch                         */
    float *z;          /* [d_inner]       host scratch                                */
    float *ffn_buf;    /* [n_ff]          host scratch                                */
    float *attn_out;   /* [n_head*head_dim] host scratch                              */
    float *logits;     /* [vocab]         last single-token / MTP logits              */
    float *scores;     /* [n_head][n_ctx] host scratch                                */

    float *rope_cos, *rope_sin;   /* [n_ctx][rope_dim/2], host copies of the device tables */
    void  *arena;

    float *bx, *bxb, *bqkv, *bkv, *bz, *bffn, *battn_out;   /* [8][...] host scratch */
    float *h_save;     /* [8][n_embd]     pre-norm hidden per token of the last batch */
    float *logits_b;   /* [8][vocab]      logits of the last batched forward          */
    void  *arena_b;

    /* rollback checkpoints: a ring of state slots in GPU memory here, NULL */
    float *ckpt_conv;
    float *ckpt_ssm;

    qwen_layer_t   mtp_layer;
    const gguf_tensor_info_t *mtp_eh_proj, *mtp_enorm, *mtp_hnorm, *mtp_shnorm;

    uint32_t n_ctx;
    uint32_t pos;

    int      host_sync;    /* 1: copy results into the fields above after each call */
    qwen_gpu_t *gpu;
} qwen_model_t;

#define SPEC_MAX_B    8    /* k = SPEC_MAX_B - 1 drafts (reference: 3, model.h:113) */
#define PREFILL_MAX_B 8    /* tokens per batched prefill chunk (model.h:114)        */

/* Loads a GGUF file and uploads it to device 0 (reference model.c:55-290).
 * 0 on success, -1 with a message on stderr. */
int  model_init(qwen_model_t *m, const char *path, uint32_t n_ctx);
/* Same for a deterministic random-init model (no file; include/qwen_synth.h). */
int  model_init_synth(qwen_model_t *m, const qwen_synth_spec_t *spec, uint32_t n_ctx);
void model_free(qwen_model_t *m);

/* single-token layers on m->x (reference model.c:418-485, :617-695) */
void attention_layer(qwen_model_t *m, qwen_layer_t *L, pool_t *pool, uint32_t pos);
void gdn_layer(qwen_model_t *m, qwen_layer_t *L, pool_t *pool);

/* single-token decode step: logits of `token` at `pos` into m->logits; pos = pos + 1
 * (reference model.c:714-744) */
void model_forward(qwen_model_t *m, pool_t *pool, uint32_t token, uint32_t pos);
/* batched forward of B <= 8 tokens at pos..pos+B-1: logits_b, h_save; pos += B
 * (reference model.c:976-1002).  ckpt is accepted for compatibility: per-token
 * state snapshots are always kept, so model_rollback_to works after any batch. */
void model_forward_batch(qwen_model_t *m, pool_t *pool, const uint32_t *tokens, uint32_t pos, uint32_t B, int ckpt);

int  model_snapshot_states(qwen_model_t *m);             /* no-op, as the reference (model.c:1004) */
void model_rollback_states(qwen_model_t *m);             /* no-op (model.c:1009) */
/* recurrent states = state after token b of the last batched forward (model.c:1015-1031);
 * the caller sets m->pos.  b must be below that forward's B (and below 8): otherwise the
 * call is ignored with a message and qwen_model_status() reports -1. */
void model_rollback_to(qwen_model_t *m, uint32_t b);

/* Start a new sequence on a loaded model (no reference counterpart: the
 * reference loads a fresh model per run): recurrent states zeroed, ring index
 * and position 0.  KV rows are overwritten before they are read. */
void model_reset(qwen_model_t *m);

/* MTP draft layer (reference model.c:1038-1063): token at pos with m->mtp_h;
 * m->mtp_h = output; logits into m->logits when want_logits.  Returns 0. */
int  mtp_forward(qwen_model_t *m, pool_t *pool, uint32_t token, uint32_t pos, int want_logits);
/* batched MTP prefill pairing tokens[b] with h_save[b] (model.c:1069-1103) */
int  mtp_forward_batch(qwen_model_t *m, pool_t *pool, const uint32_t *tokens, uint32_t pos, uint32_t B,
                       int want_logits);

/* greedy argmax over host logits, lowest index on ties (model.c:746-756) */
uint32_t model_sample_greedy(const float *logits, uint32_t vocab_size);

/* ------------------------------------------------------------------------
 * Device-resident generation (no reference counterpart: the reference runs
 * its spec loop in main.c:133-231 on host logits; this runs the same loop with
 * drafts, verification, argmax and acceptance on the GPU and returns tokens).
 * ------------------------------------------------------------------------ */
typedef struct {
    uint64_t n_cycles, n_accepted, n_drafts;
    double   t_prefill_s, t_decode_s;
} qwen_gen_stats_t;

/* Prefill (chunks of 8 + MTP prefill when k > 0), then greedy MTP speculative
 * decode with k drafts per cycle (k = 0: plain greedy decode).  force_accept
 * fixes the accepted count instead of comparing drafts with the verify argmax:
 * 1 = every draft accepted (j = k, the all-accepted throughput mode), 2 = j
 * cycles through 0, 1, .., k (exercises every rollback depth); the stream is
 * then not the greedy one.  cycle_j (optional) receives j of each cycle.
 * Returns the number of tokens written to out (<= n_predict). */
uint32_t model_generate_spec(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                             uint32_t k, uint32_t eos, int force_accept, uint32_t *out, uint32_t *cycle_j,
                             qwen_gen_stats_t *st);
/* The same loop in two parts, for callers that time or pace the cycles:
 * model_spec_begin prefills the prompt (0, or -1 on bad arguments) and, with
 * host_sync on, leaves the last prompt row's logits in m->logits (main.c:146-150);
 * model_spec_run continues from the current state for at most max_cycles
 * cycles / max_tokens tokens and may be called again to go on.  It stops as
 * main.c:210 does once the verified positions reach n_ctx.  With host_sync on,
 * it leaves logits_b / h_save (the last verify's rows; row cycle_j[last] is
 * the logits the next cycle starts from) and mtp_h in the host fields. */
int      model_spec_begin(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t k);
uint32_t model_spec_run(qwen_model_t *m, uint32_t k, uint32_t eos, int force_accept, uint32_t max_cycles,
                        uint32_t max_tokens, uint32_t *out, uint32_t *cycle_j, qwen_gen_stats_t *st);
/* Sampled decode (main.c:232-248): prefill, then every token drawn by the
 * reference sampler (sampler_init(temp, top_p, top_k, repeat_penalty, seed) +
 * sampler_sample over the prompt and the tokens generated so far), here on the
 * device (qgpu_sample), then a model_forward step.  Stops after n_predict tokens,
 * at eos (written) or at n_ctx.  Returns the number of tokens written to out. */
uint32_t model_generate_sample(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                               float temp, float top_p, uint32_t top_k, float repeat_penalty, uint64_t seed,
                               uint32_t eos, uint32_t *out, qwen_gen_stats_t *st);
/* Plain greedy decode with model_forward steps (the lossless reference stream). */
uint32_t model_generate_greedy(qwen_model_t *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_predict,
                               uint32_t eos, uint32_t *out, qwen_gen_stats_t *st);
/* One timed verify step (B tokens at the current position) and one timed decode
 * step, on device buffers (benchmark support); the model state is restored.  If the
 * last forward kept its recurrent states in factor form, the selected state is
 * written out first, and model_rollback_to is refused until the next forward. */
int  model_time_steps(qwen_model_t *m, uint32_t B, int reps, float *ms_verify, float *ms_decode, float *ms_draft);

/* Status of the last model call: 0 = done, -1 = rejected on the host (bad
 * arguments, positions past n_ctx), -2 = a device error (sticky: from then on
 * every call does nothing and returns -1 / leaves the results untouched).
 * No reference counterpart. */
int qwen_model_status(const qwen_model_t *m);

/* FFI helpers (no reference counterpart; for callers that do not mirror the
 * struct layout, e.g. ctypes): allocation and field access. */
qwen_model_t *qwen_model_alloc(void);
void          qwen_model_dealloc(qwen_model_t *m);
float        *qwen_model_field(qwen_model_t *m, const char *name);   /* "logits", "logits_b", "h_save", "mtp_h", "x" */
uint32_t      qwen_model_get(const qwen_model_t *m, const char *name); /* "pos", "vocab", "n_embd", "n_ctx", "n_layer" */
void          qwen_model_set_pos(qwen_model_t *m, uint32_t pos);
void          qwen_model_set_host_sync(qwen_model_t *m, int on);
/* 1: the launch sequences of the forward and MTP bodies are captured once as
 * HIP graphs and replayed (default 0; environment QWEN_GRAPHS=1 sets 1) */
void          qwen_model_set_graphs(qwen_model_t *m, int on);

/* 1: model_forward times its sections on the device (below).  Default: on when
 * QWEN_PROFILE is set (not "0") in the environment at model_init, the run-time
 * form of the reference's compile-time QWEN_PROFILE (model.c:701-712). */
void          qwen_model_set_profile(qwen_model_t *m, int on);

/* Profiling counters (reference model.h:151-152, accumulated by model_forward as
 * in model.c:714-742): seconds of device time per section -- the embedding row,
 * the GDN layers, the attention layers, the output norm + lm_head -- between HIP
 * events recorded on the library stream.  qwen_prof_calls counts model_forward
 * calls; the sections stay 0 while profiling is off, as in a reference build
 * without QWEN_PROFILE. */
extern double qwen_prof_embed, qwen_prof_gdn, qwen_prof_attn, qwen_prof_head;
extern uint64_t qwen_prof_calls;

#ifdef __cplusplus
}
#endif
#endif
