/*
 * qgpu.h -- C-ABI of the MI355X (gfx950) HIP layer.
 *
 * Plain C types only.  Every compute entry point takes DEVICE pointers, is
 * enqueued on the library's stream and returns immediately (stream order);
 * qgpu_sync() waits.  Return value: QGPU_OK (0), a negative QGPU_E* for a
 * rejected argument, or a positive hipError_t from the runtime.
 *
 * Each entry point names the reference function it replaces (file:line
 * relative to the reference checkout).  The C11 host library (host/ sources)
 * implements the reference's own API (include/kernels.h, include/model.h)
 * on top of these.
 */
#ifndef QGPU_H
#define QGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QGPU_OK          0
#define QGPU_E_ARG      -1    /* bad pointer / size / shape */
#define QGPU_E_TYPE     -2    /* unsupported ggml type */
#define QGPU_E_INIT     -3    /* qgpu_init not called / no device */
#define QGPU_E_RANGE    -4    /* size beyond a documented maximum */

#define QGPU_MAX_B       8    /* columns per batched GEMV (reference GEMV_MAX_B, kernels.h:19) */
#define QGPU_MAX_MULTI   8    /* matrices per grouped GEMV (reference GEMV_MULTI_MAX, kernels.c:657) */
#define QGPU_MAX_KS     32    /* K ranges per tile of a per-matrix split (qgpu_gemv_act_batch_ks) */

/* ------------------------------------------------------------ runtime */
/* Selects the device, creates the stream and the GEMV workspace. Idempotent. */
int  qgpu_init(int device);
/* Device name, compute-unit count and HBM bytes of the current device. */
int  qgpu_device_info(char *name, int name_cap, int *n_cu, uint64_t *hbm_bytes);
const char *qgpu_strerror(int status);
int  qgpu_sync(void);
int  qgpu_malloc(void **ptr, size_t bytes);
int  qgpu_free(void *ptr);
int  qgpu_memcpy_h2d(void *dst, const void *src, size_t bytes);     /* synchronous */
int  qgpu_memcpy_d2h(void *dst, const void *src, size_t bytes);     /* synchronous */
int  qgpu_memcpy_d2d(void *dst, const void *src, size_t bytes);     /* stream-ordered */
/* Pinned host memory that kernels can write (hipHostMalloc, coherent): the host sees
 * their stores without a copy.  qgpu_host_free waits for the library stream first. */
int  qgpu_host_malloc(void **p, size_t bytes);
int  qgpu_host_free(void *p);
int  qgpu_memset(void *dst, int value, size_t bytes);               /* stream-ordered */
/* Timing on the library stream (HIP events). */
int  qgpu_event_create(void **ev);
int  qgpu_event_destroy(void *ev);
int  qgpu_event_record(void *ev);
int  qgpu_event_elapsed_ms(void *start, void *stop, float *ms);     /* waits for stop */
/* HIP graph capture of the library stream. */
int  qgpu_graph_begin(void);
int  qgpu_graph_end(void **graph_exec);
int  qgpu_graph_launch(void *graph_exec);
int  qgpu_graph_destroy(void *graph_exec);

/* ------------------------------------------------------------ weights */
typedef struct qgpu_tensor qgpu_tensor;   /* device-resident weight matrix */

/* Uploads ne1 rows of ne0 elements in ggml format `type` (F32, Q8_0, Q4_K,
 * Q5_K, Q6_K, IQ4_XS; host bytes in GGUF row-major layout).  IQ4_XS is
 * repacked losslessly into 16-row tiles for the matrix-core kernel; the other
 * formats keep the GGUF layout.  Replaces binding gguf_tensor_info_t.data
 * (reference gguf.h:63-70) for GPU use. */
int  qgpu_tensor_upload(const void *host, int type, uint64_t ne0, uint64_t ne1, qgpu_tensor **out);
/* Same from bytes already in device memory (GGUF layout). */
int  qgpu_tensor_from_device(const void *dev, int type, uint64_t ne0, uint64_t ne1, qgpu_tensor **out);
int  qgpu_tensor_free(qgpu_tensor *t);
/* Rebuilds the GGUF-layout bytes (inverse of the repack) into host memory. */
int  qgpu_tensor_download(const qgpu_tensor *t, void *host);
int  qgpu_tensor_shape(const qgpu_tensor *t, int *type, uint64_t *ne0, uint64_t *ne1);
/* Bytes of the matrix in its format (algorithmic bytes, = GGUF size). */
uint64_t qgpu_tensor_bytes(const qgpu_tensor *t);

/* ------------------------------------------------------------ GEMV */
#define QGPU_GEMV_ACCUM  1    /* out += W x  instead of out = W x (fused residual add) */

/* out[t*ldo + r] (+)= sum_i W[r,i] * x[t*ldx + i] for t < n <= 8, r < ne1.
 * Replaces gemv_batch / gemv_rows_batch (reference kernels.c:570-648) and,
 * with n = 1, gemv (kernels.c:615-621). */
int  qgpu_gemv_batch(const qgpu_tensor *W, const float *x, uint64_t ldx, int n,
                     float *out, uint64_t ldo, int flags);
/* qgpu_gemv_batch without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as qgpu_gemv_batch (bit-identical), plus the HIP stream
 * to launch on (NULL: the default stream); it neither initialises the library
 * nor allocates: the activation workspace is a static device array of
 * 1,875,968 bytes per GPU (ne0 <= 65536, else QGPU_E_RANGE).  Calls that
 * overlap on one GPU share that array and race. */
int  qgpu_gemv_batch_noalloc(const qgpu_tensor *W, const float *x, uint64_t ldx, int n, float *out,
                             uint64_t ldo, int flags, void *stream);
/* Several matrices sharing x, one launch per format group.
 * Replaces gemv_multi_batch / gemv_multi (reference kernels.c:666-736). */
int  qgpu_gemv_multi_batch(const qgpu_tensor *const *Ws, int n_mat, const float *x, uint64_t ldx,
                           int n, float *const *outs, const uint64_t *ldos, int flags);
/* Split form of the matrix-core path: qgpu_gemv_prepare converts the activations
 * once (x: n rows of ne0 floats) and qgpu_gemv_prepared runs a packed matrix
 * (IQ4_XS, Q4_K, Q5_K, Q6_K or Q8_0 with ne0 % 256 == 0; QGPU_E_TYPE otherwise)
 * with ne0 columns on them; several matrices may follow one prepare. */
int  qgpu_gemv_prepare(const float *x, uint64_t ldx, int n, uint64_t ne0);
int  qgpu_gemv_prepared(const qgpu_tensor *W, int n, float *out, uint64_t ldo, int flags);
/* Fused activation transforms.  The GEMV input is computed from the rows
 * named here inside the kernel that prepares the activations, so the
 * normalisation / gating pass of the reference is not a kernel of its own:
 *   QGPU_ACT_COPY       v = x
 *   QGPU_ACT_RMSNORM    v = x / sqrt(mean(x^2) + eps) * w          (model.c:433,460,737,996)
 *                       with seg = ne0 / 2: the two halves [x | y] each
 *                       normalised with their own row and weight (w, w2):
 *                       the MTP input concat(enorm(e), hnorm(h)) (model.c:1046-1050)
 *   QGPU_ACT_SILU_MUL   v = silu(x) * y                            (model.c:477-480)
 *   QGPU_ACT_GATED_NORM v = rmsnorm_head(x) * w[i % seg] * silu(y)  per head of seg
 *                       in {64, 128, 256} elements                  (model.c:928-941)
 * xout (optional, ldxo) receives v in fp32; it is required when a matrix of
 * the call is not IQ4_XS (those kernels read fp32 rows).  ne0 % 256 == 0.
 * Single-segment QGPU_ACT_RMSNORM inside a GEMV call is computed as
 * s * (W (x w)) with s = 1/sqrt(mean(x^2) + eps) applied to the GEMV output,
 * so xout then holds x * w (the row factor is not in it).  The two-segment form
 * with no xout, before matrix-core matrices only and no K split, is computed the
 * same way with one factor per half (the MTP input's enorm and hnorm).
 * Pending K-split partial sums (qgpu_gemv_act_split): with n_part > 0 the
 * RMSNORM input is x_eff = x + sum_{q < n_part} part[q*n*ldp + t*ldp + i];
 * xnew (ldxn; may equal x) receives x_eff.  Single-segment RMSNORM only.
 * Embedding gather: with embd (a packed IQ4_XS matrix) and tok (n device token ids),
 * QGPU_ACT_RMSNORM reads row t of x (of its first segment in the two-segment form) as
 * row tok[t] of embd, dequantised as qgpu_dequant_rows does (bit-identical; ids past the
 * last row give zero rows); x is unused, embd's ne0 is the segment length, n_part is 0,
 * and the single-segment form writes the rows to xnew when set.  (The reference's
 * embedding lookups, model.c:721,982,1045,1079, in the first preparation of a forward.) */
#define QGPU_ACT_COPY        0
#define QGPU_ACT_RMSNORM     1
#define QGPU_ACT_SILU_MUL    2
#define QGPU_ACT_GATED_NORM  3
typedef struct {
    int          kind;
    const float *x;   uint64_t ldx;
    const float *y;   uint64_t ldy;
    const float *w;
    const float *w2;
    uint64_t     seg;
    float        eps;
    float       *xout; uint64_t ldxo;
    const float *part; uint64_t ldp; int n_part;
    float       *xnew; uint64_t ldxn;
    const qgpu_tensor *embd; const uint32_t *tok;
} qgpu_act;
/* qgpu_gemv_multi_batch with the input given as a transform of device rows. */
int  qgpu_gemv_act_batch(const qgpu_tensor *const *Ws, int n_mat, const qgpu_act *act, int n,
                         float *const *outs, const uint64_t *ldos, int flags);
/* qgpu_gemv_act_batch with a K split per matrix (no reference counterpart: a
 * scheduling form of the grouped GEMV, kernels.c:657).  The tiles of matrix j
 * are cut into ks[j] K ranges (1..QGPU_MAX_KS, at most ne0 / 256), and range q
 * writes partial plane q: outs[j][q*n*ldos[j] + t*ldos[j] + r]; the caller sums
 * the planes in q order (ks[j] = 1: the plain output).  Splitting the small
 * matrices of a grouped launch spreads their bytes over many compute units
 * instead of adding a whole tile to a few.  Packed formats for ks[j] > 1; no
 * accumulation. */
int  qgpu_gemv_act_batch_ks(const qgpu_tensor *const *Ws, int n_mat, const qgpu_act *act, int n,
                            float *const *outs, const uint64_t *ldos, const int *ks);
/* Transform only: v into act->xout (required) and the IQ4_XS digit planes
 * (so qgpu_gemv_prepared may follow). */
int  qgpu_act_prepare(const qgpu_act *act, int n, uint64_t ne0);
/* K-split form for narrow outputs (ne1 rows spread over too few tiles to load
 * every compute unit): ks blocks per 16-row tile each reduce one K range and
 * write partial plane q: part[q*n*ldp + t*ldp + r] (no accumulation).  The
 * planes are summed, in q order, by the next QGPU_ACT_RMSNORM that names them
 * (n_part = ks) or by qgpu_add_partials.  IQ4_XS only; ks in 1..8. */
int  qgpu_gemv_act_split(const qgpu_tensor *W, const qgpu_act *act, int n, float *part, uint64_t ldp, int ks);
/* ks that balances W over the device's compute units (1: no split). */
int  qgpu_gemv_split_ks(const qgpu_tensor *W);
/* qgpu_gemv_act_split on the input already prepared by qgpu_gemv_prepare,
 * qgpu_act_prepare or qgpu_attn_fused_act (packed W only). */
int  qgpu_gemv_prepared_split(const qgpu_tensor *W, int n, float *part, uint64_t ldp, int ks);
/* rows x n: y = x + sum_{q < n_part} part[q*rows*ldp + r*ldp + i] (y may equal x). */
int  qgpu_add_partials(float *y, uint64_t ldy, const float *x, uint64_t ldx, const float *part, uint64_t ldp,
                       int n_part, uint64_t n, int rows);
/* Rows [r0, r1) only (reference gemv_rows, kernels.c:298-321). */
int  qgpu_gemv_rows_batch(const qgpu_tensor *W, const float *x, uint64_t ldx, int n,
                          float *out, uint64_t ldo, uint64_t r0, uint64_t r1);

/* ------------------------------------------------------------ dequant */
/* out[b*ldo + i] = dequant(row rows[b])[i] for b < n, rows in DEVICE memory.
 * Bit-exact with the reference scalar decoder (quant.c:86-208); replaces the
 * embedding fetch dequant_row(tok_embd, quant_row_ptr(tok_embd, token))
 * (reference model.c:721,982,1045,1079). */
int  qgpu_dequant_rows(const qgpu_tensor *W, const uint32_t *rows, int n, float *out, uint64_t ldo);

/* ------------------------------------------------------------ ops (reference kernels.c:741-939) */
/* rows x n: out[r*ldo+i] = x[r*ldx+i] / sqrt(mean(x^2)+eps) * w[i]   (w may be NULL) */
int  qgpu_rmsnorm(float *out, uint64_t ldo, const float *x, uint64_t ldx, const float *w,
                  uint64_t n, int rows, float eps);
/* rows x n: out = x / max(||x||, eps) */
int  qgpu_l2norm(float *out, uint64_t ldo, const float *x, uint64_t ldx, uint64_t n, int rows, float eps);
int  qgpu_silu(float *x, uint64_t n);
int  qgpu_sigmoid(float *x, uint64_t n);
int  qgpu_softplus(float *x, uint64_t n);
/* rows x n, in place */
int  qgpu_softmax(float *x, uint64_t ld, uint64_t n, int rows);
/* rows x n: a[r*lda+i] = silu(a[r*lda+i]) * b[r*ldb+i]   (FFN gate, model.c:477-480) */
int  qgpu_silu_mul(float *a, uint64_t lda, const float *b, uint64_t ldb, uint64_t n, int rows);
/* rows x n: y[r*ldy+i] += x[r*ldx+i]  (residual add) */
int  qgpu_add(float *y, uint64_t ldy, const float *x, uint64_t ldx, uint64_t n, int rows);
/* device copy kernel (16-byte aligned, multiple of 16 bytes); graph-capturable */
int  qgpu_copy(void *dst, const void *src, size_t bytes);
/* Plain read of src (16-byte aligned, a multiple of 16 bytes) by n blocks
 * (1..65536): block b writes to partials[b] (device) the XOR of the 32-bit words
 * of its share, so the XOR of partials[0..n) is the XOR of every word of src.
 * Stream-ordered, graph-capturable.  For device-memory integrity checks against
 * a host XOR, and as the read-bandwidth floor the GEMV kernels are measured
 * against (n = 2048).  No counterpart in the reference (no device memory there). */
int  qgpu_checksum(const void *src, size_t bytes, uint32_t *partials, int n);
/* qgpu_checksum over a tensor's device bytes: the tile records of the matrix-core
 * formats, the GGUF rows of the others (qgpu_tensor_device_bytes of them) */
int  qgpu_tensor_checksum(const qgpu_tensor *t, uint32_t *partials, int n);
uint64_t qgpu_tensor_device_bytes(const qgpu_tensor *t);
/* argmax of each of `rows` rows (lowest index wins ties; model.c:746-756) into out[r] */
int  qgpu_argmax(const float *logits, uint64_t ld, uint32_t n, int rows, uint32_t *out);

/* ------------------------------------------------------------ Gated DeltaNet (model.c:494-615,845-941) */
/* Recurrent state is kept in a ring of `nslot` slots of `slot_stride` floats:
 * the current state is slot *cur (device int); the state after token b of a
 * batch goes to slot (*cur + 1 + b) % nslot.  Rolling back to the state after
 * token j (reference model_rollback_to, model.c:1015-1031) is *cur = (*cur+1+j) % nslot. */
/* causal conv1d (4 taps) + SiLU of B <= 8 tokens: y[b] = silu(conv(state, x[b])) (model.c:891-909) */
int  qgpu_gdn_conv(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w, float *ring,
                   uint64_t slot_stride, int nslot, const int *cur, float *y, uint64_t ldy);
/* per-k-head L2 norm of q,k and the delta-rule recurrence over B tokens for all
 * n_v v-heads (v-head h reads k-head h % n_k), head_dim 128 (model.c:494-595) */
int  qgpu_gdn_recurrence(const float *xq, uint64_t ldq, const float *beta_raw, const float *alpha_raw,
                         uint64_t ldba, const float *dt_bias, const float *ssm_a, float *ring,
                         uint64_t slot_stride, int nslot, const int *cur, int B, int n_k, int n_v,
                         int head_dim, float eps, float *out, uint64_t ldo);
/* qgpu_gdn_conv + qgpu_gdn_recurrence in one launch (same arguments, results
 * and ring slots; the conv output is not stored): conv_dim = (2 n_k + n_v) * 128,
 * x = the raw wqkv projection rows. */
int  qgpu_gdn_fused(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w, float *conv_ring,
                    uint64_t conv_stride, const float *beta_raw, const float *alpha_raw, uint64_t ldba,
                    const float *dt_bias, const float *ssm_a, float *ssm_ring, uint64_t ssm_stride, int nslot,
                    const int *cur, int n_k, int n_v, int head_dim, float eps, float *out, uint64_t ldo);
/* qgpu_gdn_fused with beta_raw and alpha_raw given as ba_planes partial planes
 * (plane q at beta_raw + q*ba_pstride, the same for alpha_raw; 1..QGPU_MAX_KS,
 * ba_planes * B <= 256), summed in plane order per token and head: the outputs
 * of qgpu_gemv_act_batch_ks. */
int  qgpu_gdn_fused_planes(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w, float *conv_ring,
                           uint64_t conv_stride, const float *beta_raw, const float *alpha_raw, uint64_t ldba,
                           int ba_planes, uint64_t ba_pstride, const float *dt_bias, const float *ssm_a,
                           float *ssm_ring, uint64_t ssm_stride, int nslot, const int *cur, int n_k, int n_v,
                           int head_dim, float eps, float *out, uint64_t ldo);
/* qgpu_gdn_fused_planes with the recurrent state kept in rank-1 factor form
 * (the same recurrence as model.c:494-615; the reference keeps snapshots,
 * model.c:1015-1031).  The state after token b is dec_b * S_{b-1} + d_b kn_b^T
 * per v-head (d_b: one coefficient per state row, kn_b: the normalised k of its
 * k-head, dec_b: the decay), exactly the update the recurrence applies.
 * factors: two buffers of 8 token records of f_tok floats each (f_tok >=
 * (n_v + n_k) * 128 + n_v, a multiple of 4): record b = d_b of every v-head
 * [n_v][128], then kn_b [n_k][128], then dec_b [n_v].  fstate (device, 2 ints):
 * P, the tokens of the previous factor-form call still to be applied, and the
 * buffer holding their factors.  The call reads the state in slot
 * (*cur - P) % nslot and applies those P tokens first; factor_out = 0: it then
 * writes the state after each of its B tokens to slot (*cur + 1 + b) % nslot as
 * qgpu_gdn_fused_planes does; factor_out = 1: it writes the state after the P
 * tokens to slot *cur and the factors of its B tokens to the other buffer, and
 * no state snapshots.  After a factor_out = 1 call at slot c, rolling back to
 * the state after token j is *cur = (c + 1 + j) % nslot with P = j + 1 and the
 * buffer flipped; the conv states are snapshots in both forms.  fstate = NULL
 * and factor_out = 0 is qgpu_gdn_fused_planes.  No reference counterpart:
 * the verify writes one state instead of B. */
int  qgpu_gdn_fused_factor(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w, float *conv_ring,
                           uint64_t conv_stride, const float *beta_raw, const float *alpha_raw, uint64_t ldba,
                           int ba_planes, uint64_t ba_pstride, const float *dt_bias, const float *ssm_a,
                           float *ssm_ring, uint64_t ssm_stride, int nslot, const int *cur, int n_k, int n_v,
                           int head_dim, float eps, float *out, uint64_t ldo, float *factors, uint64_t f_tok,
                           const int *fstate, int factor_out);
/* the state after the P pending tokens of fstate (see qgpu_gdn_fused_factor) into slot *cur */
int  qgpu_gdn_materialize(float *ssm_ring, uint64_t ssm_stride, int nslot, const int *cur, int n_k, int n_v,
                          int head_dim, const float *factors, uint64_t f_tok, const int *fstate);
/* rows x n: out = rmsnorm(x, w) * silu(z)  (per-head gated norm, model.c:928-941) */
int  qgpu_rmsnorm_gated(float *out, const float *x, const float *z, const float *w, int n, int rows,
                        uint64_t ld, float eps);

/* ------------------------------------------------------------ attention (model.c:318-406,760-810) */
/* q: [B][n_head*2*head_dim] (q | gate per head) normed + RoPE'd in place; k, v:
 * [B][n_kv*head_dim]; k normed + RoPE'd and v written to the caches at row
 * *pos_dev + b.  RoPE tables [n_ctx][rope_dim/2] (cos, sin). head_dim 256. */
int  qgpu_attn_prep(float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                    const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                    const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev, int B,
                    int n_head, int n_kv, int head_dim, float eps);
/* out[b][h*hd+d] = (softmax_{t <= pos+b}(q_bh . k_t / sqrt(hd)) V)[d] * sigmoid(gate_bh[d]);
 * ctx_bound >= pos + B bounds the positions read (spans beyond *pos_dev+B-1 exit).
 * (n_head/n_kv)*B <= 48. */
int  qgpu_attn_decode(const float *q, uint64_t ldq, const float *kcache, const float *vcache,
                      const int *pos_dev, int ctx_bound, int B, int n_head, int n_kv, int head_dim,
                      float *out, uint64_t ldo);
/* qgpu_attn_prep + qgpu_attn_decode in fewer launches: the per-head q/k
 * RMSNorm, RoPE and the cache writes of the B new rows happen inside the
 * attention kernel.  q is not modified.  Same arguments and results as the
 * two calls (model.c:318-406, 760-810); B <= 8. */
int  qgpu_attn_fused(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                     const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                     const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev,
                     int ctx_bound, int B, int n_head, int n_kv, int head_dim, float eps, float *out, uint64_t ldo);
/* qgpu_attn_fused whose output rows are also prepared as the input of the next
 * GEMV: the digit planes of out (n_head*head_dim columns) are written exactly as
 * qgpu_act_prepare with QGPU_ACT_COPY would write them from out, so
 * qgpu_gemv_prepared or qgpu_gemv_prepared_split may follow with no preparation
 * launch (the o-projection input, model.c:811-816).  out may be NULL: then only the
 * digit planes are written. */
int  qgpu_attn_fused_act(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                         const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                         const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev,
                         int ctx_bound, int B, int n_head, int n_kv, int head_dim, float eps, float *out, uint64_t ldo);
/* qgpu_attn_fused_act for a caller that knows a bound on the live context: live_hi >= pos + B
 * for every position the launch will see (a captured graph's replays included).  While
 * live_hi <= qgpu_attn_split_bound(ctx_bound, B, n_head, n_kv), the span blocks of each kv
 * head are doubled, each serving half of its query heads; the results are bit-identical to
 * qgpu_attn_fused_act.  live_hi = 0: no bound (qgpu_attn_fused_act); QGPU_E_ARG when
 * 0 < live_hi < B or live_hi > ctx_bound.  (No reference counterpart: the reference's
 * attention loops over heads on the CPU, model.c:353-406.) */
int  qgpu_attn_fused_act_live(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                              const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                              const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev,
                              int ctx_bound, int B, int n_head, int n_kv, int head_dim, float eps, float *out,
                              uint64_t ldo, int live_hi);
/* The largest live context (positions, <= ctx_bound) up to which qgpu_attn_fused_act_live splits
 * the query heads of B tokens over two blocks per span; 0 when it never does (where the split
 * would not take fewer 16-row tiles, e.g. B = 1 or 2 with 6 query heads per kv head).
 * Initialises the library when needed. */
int  qgpu_attn_split_bound(int ctx_bound, int B, int n_head, int n_kv);
/* allocates the attention workspace for ctx_bound positions now (no allocation later);
 * QGPU_E_RANGE when the KV cache does not fit the kernels' offsets (qgpu_attn_cache_fits) */
int  qgpu_attn_reserve(int ctx_bound, int n_kv);
/* 1 when a KV cache of ctx_bound positions x n_kv heads (head_dim 256, fp32) lies within the
 * attention kernels' 32-bit buffer offsets (ctx_bound * n_kv * 1024 bytes <= 2^31 - 1), else 0.
 * The attention calls and qgpu_attn_reserve return QGPU_E_RANGE beyond it; model_init refuses
 * such an n_ctx.  Arithmetic only: no device work, callable without a GPU.  (No reference
 * counterpart: the reference's KV cache is host memory with 64-bit indexing.) */
int  qgpu_attn_cache_fits(int ctx_bound, int n_kv);

/* ------------------------------------------------------------ sampling (sampler.c:62-162) */
/* sampler_sample on device data: logits[vocab] (the repeat penalty is applied in
 * place, as the reference does), tokens[n_tokens] the prompt and generated
 * tokens (the last repeat_last_n are penalised), *rng_state the xorshift64 state
 * (advanced once per non-greedy call), *out_token the chosen id.  temp, top_p,
 * top_k, repeat_penalty, repeat_last_n: the fields of an initialised sampler_t
 * (top_k >= 1; top_k > 256 takes 256).  temp <= 0 or top_k == 1: the first
 * maximum, and rng_state may be NULL.  QGPU_E_RANGE for vocab > 2^24 or a
 * penalty window of more than 4096 tokens.  Stream-ordered; the first call for
 * a larger vocabulary or top_k allocates the candidate buffers.  Logits of
 * exactly equal value are taken in index order (the reference's order among
 * them follows its heap and qsort). */
int  qgpu_sample(float *logits, uint32_t vocab, const uint32_t *tokens, uint32_t n_tokens, float temp,
                 float top_p, uint32_t top_k, float repeat_penalty, uint32_t repeat_last_n,
                 uint64_t *rng_state, uint32_t *out_token);

/* ------------------------------------------------------------ driver helpers */
/* *dst = value, stream-ordered (graph-capturable) */
int  qgpu_set_i32(int *dst, int value);
/* Greedy acceptance of one speculative cycle (main.c:191-217) on the device:
 *   j = first i < k with vtok[i] != cand[i+1], else k  (force_j >= 0: j = min(force_j, k),
 *   the benchmark's fixed-acceptance modes; -1 for greedy acceptance);
 *   out[0] = j; out[1 .. j+1] = cand[0 .. j] (emitted tokens); out[j+2] = vtok[j] (next cand[0]);
 *   *cur = (*cur + 1 + j) % nslot (GDN rollback);  *pos += j + 1 (next position).
 * `vtok` are the argmax tokens of the B = k+1 verify rows (qgpu_argmax). */
int  qgpu_spec_accept(const uint32_t *cand, const uint32_t *vtok, int k, int force_j, int *pos, int *cur,
                      int nslot, uint32_t *out);
/* qgpu_spec_accept with the incoming position and ring slot given as values (pos0 >= 0,
 * 0 <= cur0 < nslot) instead of read from *pos / *cur: *cur = (cur0 + 1 + j) % nslot,
 * *pos = pos0 + j + 1.  Same acceptance (main.c:191-217); the caller needs no launch to
 * set them first. */
int  qgpu_spec_accept_at(const uint32_t *cand, const uint32_t *vtok, int k, int force_j, int pos0, int cur0,
                         int *pos, int *cur, int nslot, uint32_t *out);
/* qgpu_spec_accept_at that also hands the next MTP forward its inputs on the device, so
 * the caller can enqueue that forward before it reads j (main.c:219-221, the re-anchor):
 * *tok_out = cand[j] and row_out[0..n) = rows[j*ld .. j*ld+n) (h_save[j]) when non-NULL,
 * and *cand0_out = vtok[j] (the next cycle's cand[0]) when non-NULL, written after every
 * read of cand, so it may point at cand[0].  With pos0 = P, the position of the token
 * before the verified ones, *pos = P + j + 1 is the re-anchor's position.  `out` may be
 * qgpu_host_malloc memory: out[0] (j) is stored last, after a system-scope fence, so a
 * host that sees out[0] change can read out[1 .. j+2] without waiting for the stream. */
int  qgpu_spec_accept_anchor(const uint32_t *cand, const uint32_t *vtok, int k, int force_j, int pos0, int cur0,
                             int *pos, int *cur, int nslot, uint32_t *out, const float *rows, uint64_t ld, int n,
                             float *row_out, uint32_t *tok_out, uint32_t *cand0_out);

#ifdef __cplusplus
}
#endif
#endif
