/*
 * kernels_api.c -- the reference's kernels.h API (host pointers, synchronous)
 * implemented on the HIP layer.  Weights are uploaded once per data address.
 */
#include "kernels.h"
#include "qgpu.h"
#include "quant.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct { const void *key; uint64_t ne0, ne1; int type; qgpu_tensor *t; } wentry;
static wentry *g_w;
static size_t g_nw, g_cap;

/* The reference functions return nothing and write zeros for a weight type
 * they do not support (kernels.c:596).  Here any failure (unsupported type,
 * allocation, device error) is reported once on stderr, leaves zeros in the
 * requested outputs, and is kept for kernels_status(). */
static int g_status;

static int fail(const char *what, int rc)
{
    if (!g_status) fprintf(stderr, "qwen gpu: %s failed: %s\n", what, qgpu_strerror(rc));
    g_status = rc ? rc : QGPU_E_ARG;
    return -1;
}

int kernels_status(void) { return g_status; }

static qgpu_tensor *weight(const gguf_tensor_info_t *W)
{
    for (size_t i = 0; i < g_nw; i++)
        if (g_w[i].key == W->data && g_w[i].ne0 == W->ne[0] && g_w[i].ne1 == W->ne[1] && g_w[i].type == (int)W->type)
            return g_w[i].t;
    qgpu_tensor *t = NULL;
    const uint64_t rows = W->n_dims >= 2 ? W->ne[1] : 1;
    int rc = qgpu_tensor_upload(W->data, (int)W->type, W->ne[0], rows, &t);
    if (rc) { fail("weight upload", rc); return NULL; }
    if (g_nw == g_cap) {
        wentry *nw = realloc(g_w, (g_cap ? 2 * g_cap : 64) * sizeof *g_w);
        if (!nw) { qgpu_tensor_free(t); fail("host allocation", QGPU_E_ARG); return NULL; }
        g_w = nw;
        g_cap = g_cap ? 2 * g_cap : 64;
    }
    g_w[g_nw++] = (wentry){ W->data, W->ne[0], rows, (int)W->type, t };
    return t;
}

void kernels_release_weights(void)
{
    for (size_t i = 0; i < g_nw; i++) qgpu_tensor_free(g_w[i].t);
    free(g_w);
    g_w = NULL;
    g_nw = g_cap = 0;
}

/* device staging buffers, grown on demand */
static float *dev_buf(int slot, size_t bytes)
{
    static float *p[4];
    static size_t cap[4];
    if (bytes > cap[slot]) {
        if (p[slot]) qgpu_free(p[slot]);
        p[slot] = NULL;
        cap[slot] = 0;
        int rc = qgpu_malloc((void **)&p[slot], bytes);
        if (rc) { p[slot] = NULL; fail("device allocation", rc); return NULL; }
        cap[slot] = bytes;
    }
    return p[slot];
}

/* activations packed densely on the device: rows of ne0 floats, 16-byte aligned rows */
static float *stage_x(const float *x, uint64_t ldx, int n, uint64_t ne0, uint64_t *ld_dev)
{
    const uint64_t ld = (ne0 + 3) & ~(uint64_t)3;
    float *d = dev_buf(0, (size_t)n * ld * sizeof(float));
    if (!d) return NULL;
    if (ld == ldx && ld == ne0) {
        int rc = qgpu_memcpy_h2d(d, x, (size_t)n * ld * sizeof(float));
        if (rc) { fail("copy to device", rc); return NULL; }
    } else {
        for (int t = 0; t < n; t++) {
            int rc = qgpu_memcpy_h2d(d + (size_t)t * ld, x + (size_t)t * ldx, ne0 * sizeof(float));
            if (rc) { fail("copy to device", rc); return NULL; }
        }
    }
    *ld_dev = ld;
    return d;
}

static void zero_out(float *out, uint64_t ldo, int n, uint64_t r0, uint64_t r1)
{
    for (int t = 0; t < n; t++) memset(out + (size_t)t * ldo + r0, 0, (r1 - r0) * sizeof(float));
}

static void fetch_out(float *out, uint64_t ldo, const float *dout, uint64_t rows, int n, uint64_t r0, uint64_t r1)
{
    for (int t = 0; t < n; t++) {
        int rc = qgpu_memcpy_d2h(out + (size_t)t * ldo + r0, dout + (size_t)t * rows + r0, (r1 - r0) * sizeof(float));
        if (rc) { fail("copy to host", rc); zero_out(out, ldo, n, r0, r1); return; }
    }
}

void gemv_rows_batch(const gguf_tensor_info_t *W, const float *x, uint64_t ldx, int n, float *out, uint64_t ldo,
                     uint64_t r0, uint64_t r1)
{
    const uint64_t rows = W && W->n_dims >= 2 ? W->ne[1] : 1;
    if (!W || r1 <= r0 || n < 1) return;
    if (n > GEMV_MAX_B || r1 > rows) {
        /* the rows and tokens the caller's buffer holds within the request are zeroed */
        fail("gemv (batch above 8 or rows past the matrix)", QGPU_E_ARG);
        if (out && r0 < rows) zero_out(out, ldo, n < GEMV_MAX_B ? n : GEMV_MAX_B, r0, r1 < rows ? r1 : rows);
        return;
    }
    qgpu_tensor *T = weight(W);
    if (!T) { zero_out(out, ldo, n, r0, r1); return; }
    uint64_t ld = 0;
    const float *dx = stage_x(x, ldx, n, W->ne[0], &ld);
    float *dout = dx ? dev_buf(1, (size_t)n * rows * sizeof(float)) : NULL;
    int rc = dout ? qgpu_gemv_rows_batch(T, dx, ld, n, dout, rows, r0, r1) : QGPU_E_ARG;
    if (rc) { if (dout) fail("gemv", rc); zero_out(out, ldo, n, r0, r1); return; }
    fetch_out(out, ldo, dout, rows, n, r0, r1);
}

void gemv_rows(const gguf_tensor_info_t *W, const float *x, float *out, uint64_t r0, uint64_t r1)
{
    gemv_rows_batch(W, x, W->ne[0], 1, out, W->ne[1], r0, r1);
}

void gemv_batch(pool_t *pool, const gguf_tensor_info_t *W, const float *x, uint64_t ldx, int n, float *out,
                uint64_t ldo)
{
    (void)pool;
    gemv_rows_batch(W, x, ldx, n, out, ldo, 0, W->ne[1]);
}

void gemv(pool_t *pool, const gguf_tensor_info_t *W, const float *x, float *out)
{
    (void)pool;
    gemv_rows_batch(W, x, W->ne[0], 1, out, W->ne[1], 0, W->ne[1]);
}

void gemv_multi_batch(pool_t *pool, const gguf_tensor_info_t *const *Ws, const float *x, uint64_t ldx, int n,
                      float *const *outs, const uint64_t *ldos, int n_mat)
{
    (void)pool;
    for (int k = 0; k < n_mat; k++) gemv_rows_batch(Ws[k], x, ldx, n, outs[k], ldos[k], 0, Ws[k]->ne[1]);
}

void gemv_multi(pool_t *pool, const gguf_tensor_info_t *const *Ws, const float *x, float *const *outs, int n_mat)
{
    (void)pool;
    for (int k = 0; k < n_mat; k++) gemv_rows_batch(Ws[k], x, Ws[k]->ne[0], 1, outs[k], Ws[k]->ne[1], 0, Ws[k]->ne[1]);
}

/* ---------------------------------------------------------------- ops */
static void run_rows(int op, float *out, const float *x, const float *w, uint64_t n, float eps)
{
    if (!n) return;
    float *d = dev_buf(2, n * sizeof(float) * 2);
    if (!d) { memset(out, 0, n * sizeof(float)); return; }
    float *dw = d + n;
    int rc = qgpu_memcpy_h2d(d, x, n * sizeof(float));
    if (!rc && w) rc = qgpu_memcpy_h2d(dw, w, n * sizeof(float));
    if (rc) { fail("copy to device", rc); memset(out, 0, n * sizeof(float)); return; }
    switch (op) {
    case 0: rc = qgpu_rmsnorm(d, n, d, n, w ? dw : NULL, n, 1, eps); break;
    case 1: rc = qgpu_l2norm(d, n, d, n, n, 1, eps); break;
    case 2: rc = qgpu_silu(d, n); break;
    case 3: rc = qgpu_sigmoid(d, n); break;
    case 4: rc = qgpu_softplus(d, n); break;
    default: rc = qgpu_softmax(d, n, n, 1); break;
    }
    if (rc) { fail("op", rc); memset(out, 0, n * sizeof(float)); return; }
    rc = qgpu_memcpy_d2h(out, d, n * sizeof(float));
    if (rc) { fail("copy to host", rc); memset(out, 0, n * sizeof(float)); }
}

void rmsnorm(float *out, const float *x, const float *weight, uint64_t n, float eps) { run_rows(0, out, x, weight, n, eps); }
void l2norm(float *out, const float *x, uint64_t n, float eps) { run_rows(1, out, x, NULL, n, eps); }
void silu_inplace(float *x, uint64_t n) { run_rows(2, x, x, NULL, n, 0); }
void sigmoid_inplace(float *x, uint64_t n) { run_rows(3, x, x, NULL, n, 0); }
void softplus_inplace(float *x, uint64_t n) { run_rows(4, x, x, NULL, n, 0); }
void softmax_inplace(float *x, uint64_t n) { run_rows(5, x, x, NULL, n, 0); }
