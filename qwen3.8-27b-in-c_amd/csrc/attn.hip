// Gated GQA decode attention for B query tokens (gfx950); reference
// model.c:318-406 (RoPE, per-head loop) and :760-810 (batched layer).
//
//  qgpu_attn_prep   : per-head RMSNorm of q and k, NeoX partial RoPE on the
//                     first rope_dim dims (pairs (i, i + rope_dim/2)), k and v
//                     written to the cache at position pos + b.
//  qgpu_attn_decode : softmax(q K^T / sqrt(hd)) V over positions t <= pos + b,
//                     times sigmoid(gate).  Flash-decoding: one block per
//                     (kv head, 32-position chunk) serves every query head of
//                     the group and every token of the batch (each K/V row is
//                     read once per chunk), then a combine pass merges chunks.
// Positions come from device memory (*pos_dev) so the launch sequence can be
// captured in a graph and replayed at any position.
#include "qgpu_internal.h"

#define ATT_HD   256
#define ATT_CS   32
#define ATT_MAXQ 64             // query heads per kv head x batch

namespace qg {
void *ws_attn = nullptr;
size_t ws_attn_bytes = 0;
}

__global__ __launch_bounds__(ATT_HD) void k_attn_prep(float *q, uint64_t ldq, const float *k, const float *v,
                                                      uint64_t ldkv, const float *qw, const float *kw, float *kc,
                                                      float *vc, const float *rcos, const float *rsin, int half,
                                                      const int *pos_dev, int n_head, int n_kv, float eps)
{
    __shared__ float sh[ATT_HD];
    __shared__ float red[4];
    const int b = blockIdx.x, hh = blockIdx.y, t = threadIdx.x;
    const int pos = *pos_dev + b;
    const bool isq = hh < n_head;
    const int g = hh - n_head;
    float val = isq ? q[(uint64_t)b * ldq + (uint64_t)hh * 2 * ATT_HD + t] : k[(uint64_t)b * ldkv + (uint64_t)g * ATT_HD + t];
    float s = val * val;
#pragma unroll
    for (int o = 32; o; o >>= 1) s += __shfl_xor(s, o);
    if ((t & 63) == 0) red[t >> 6] = s;
    __syncthreads();
    s = red[0] + red[1] + red[2] + red[3];
    const float scale = 1.0f / sqrtf(s / (float)ATT_HD + eps);
    val = (val * scale) * (isq ? qw[t] : kw[t]);
    sh[t] = val;
    __syncthreads();
    if (t < half) {                               // rotate the pair (t, t + half)
        const float c = rcos[(uint64_t)pos * half + t], sn = rsin[(uint64_t)pos * half + t];
        const float v0 = sh[t], v1 = sh[t + half];
        sh[t] = v0 * c - v1 * sn;
        sh[t + half] = v0 * sn + v1 * c;
    }
    __syncthreads();
    if (isq) {
        q[(uint64_t)b * ldq + (uint64_t)hh * 2 * ATT_HD + t] = sh[t];
    } else {
        const uint64_t row = (uint64_t)pos * n_kv * ATT_HD + (uint64_t)g * ATT_HD + t;
        kc[row] = sh[t];
        vc[row] = v[(uint64_t)b * ldkv + (uint64_t)g * ATT_HD + t];
    }
}

// partials layout: [n_kv][nchunk][ATT_MAXQ] of (m, l) and [n_kv][nchunk][ATT_MAXQ][ATT_HD] of o
__global__ __launch_bounds__(256) void k_attn_chunk(const float *q, uint64_t ldq, const float *kc, const float *vc,
                                                    const int *pos_dev, int B, int n_head, int n_kv, int nchunk,
                                                    float *pml, float *po)
{
    __shared__ float qs[ATT_MAXQ][ATT_HD];
    __shared__ float kv[ATT_CS][ATT_HD + 1];
    __shared__ float ps[ATT_MAXQ][ATT_CS];
    const int g = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
    const int per = n_head / n_kv, QH = per * B;
    const int pos0 = *pos_dev;
    const int t0 = c * ATT_CS;
    const int tmax = pos0 + B - 1;                // last position any query may see
    float *ml = pml + ((uint64_t)g * nchunk + c) * ATT_MAXQ * 2;
    float *o = po + ((uint64_t)g * nchunk + c) * ATT_MAXQ * ATT_HD;
    if (t0 > tmax) {                              // chunk beyond the context: empty partial
        for (int qi = tid; qi < QH; qi += blockDim.x) { ml[2 * qi] = -INFINITY; ml[2 * qi + 1] = 0.0f; }
        return;
    }
    // queries qi = b * per + (h - g*per)
    for (int e = tid; e < QH * ATT_HD; e += blockDim.x) {
        const int qi = e / ATT_HD, d = e % ATT_HD, b = qi / per, h = g * per + qi % per;
        qs[qi][d] = q[(uint64_t)b * ldq + (uint64_t)h * 2 * ATT_HD + d];
    }
    const uint64_t kvrow = (uint64_t)n_kv * ATT_HD;
    for (int e = tid; e < ATT_CS * ATT_HD; e += blockDim.x) {
        const int tt = e / ATT_HD, d = e % ATT_HD, t = t0 + tt;
        kv[tt][d] = t <= tmax ? kc[(uint64_t)t * kvrow + (uint64_t)g * ATT_HD + d] : 0.0f;
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)ATT_HD);
    for (int e = tid; e < QH * ATT_CS; e += blockDim.x) {
        const int qi = e / ATT_CS, tt = e % ATT_CS, t = t0 + tt, b = qi / per;
        float s = 0.0f;
#pragma unroll 8
        for (int d = 0; d < ATT_HD; d++) s = fmaf(qs[qi][d], kv[tt][d], s);
        ps[qi][tt] = (t <= pos0 + b) ? s * scale : -INFINITY;
    }
    __syncthreads();
    // chunk softmax statistics (one wave per query row, lanes over positions)
    for (int qi = tid >> 6; qi < QH; qi += blockDim.x >> 6) {
        const int l = tid & 63;
        float v = l < ATT_CS ? ps[qi][l] : -INFINITY;
        float m = v;
#pragma unroll
        for (int off = 32; off; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float p = (l < ATT_CS && m > -INFINITY) ? expf(v - m) : 0.0f;
        float sum = p;
#pragma unroll
        for (int off = 32; off; off >>= 1) sum += __shfl_xor(sum, off);
        if (l < ATT_CS) ps[qi][l] = p;
        if (l == 0) { ml[2 * qi] = m; ml[2 * qi + 1] = sum; }
    }
    __syncthreads();
    for (int e = tid; e < ATT_CS * ATT_HD; e += blockDim.x) {
        const int tt = e / ATT_HD, d = e % ATT_HD, t = t0 + tt;
        kv[tt][d] = t <= tmax ? vc[(uint64_t)t * kvrow + (uint64_t)g * ATT_HD + d] : 0.0f;
    }
    __syncthreads();
    const int d = tid;                            // blockDim == ATT_HD
    for (int qi = 0; qi < QH; qi++) {
        float acc = 0.0f;
#pragma unroll 8
        for (int tt = 0; tt < ATT_CS; tt++) acc = fmaf(ps[qi][tt], kv[tt][d], acc);
        o[(uint64_t)qi * ATT_HD + d] = acc;
    }
}

__global__ __launch_bounds__(ATT_HD) void k_attn_combine(const float *q, uint64_t ldq, const float *pml,
                                                         const float *po, int B, int n_head, int n_kv, int nchunk,
                                                         float *out, uint64_t ldo)
{
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int per = n_head / n_kv, g = h / per, qi = b * per + (h % per);
    float m = -INFINITY;
    for (int c = 0; c < nchunk; c++) m = fmaxf(m, pml[((uint64_t)g * nchunk + c) * ATT_MAXQ * 2 + 2 * qi]);
    float l = 0.0f, acc = 0.0f;
    for (int c = 0; c < nchunk; c++) {
        const float mc = pml[((uint64_t)g * nchunk + c) * ATT_MAXQ * 2 + 2 * qi];
        if (mc == -INFINITY) continue;
        const float f = expf(mc - m);
        l += pml[((uint64_t)g * nchunk + c) * ATT_MAXQ * 2 + 2 * qi + 1] * f;
        acc += po[((uint64_t)g * nchunk + c) * ATT_MAXQ * ATT_HD + (uint64_t)qi * ATT_HD + d] * f;
    }
    const float gate = q[(uint64_t)b * ldq + (uint64_t)h * 2 * ATT_HD + ATT_HD + d];
    out[(uint64_t)b * ldo + (uint64_t)h * ATT_HD + d] = (acc / l) * (1.0f / (1.0f + expf(-gate)));
}

extern "C" int qgpu_attn_prep(float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                              const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                              const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev, int B,
                              int n_head, int n_kv, int head_dim, float eps)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (head_dim != ATT_HD) return QGPU_E_RANGE;
    if (!q || !k || !v || !q_norm_w || !k_norm_w || !kcache || !vcache || !rope_cos || !rope_sin || !pos_dev ||
        B < 1 || n_kv < 1 || n_head % n_kv || rope_dim < 2 || rope_dim > ATT_HD || rope_dim % 2)
        return QGPU_E_ARG;
    hipLaunchKernelGGL(k_attn_prep, dim3(B, n_head + n_kv), dim3(ATT_HD), 0, qg::stream, q, ldq, k, v, ldkv,
                       q_norm_w, k_norm_w, kcache, vcache, rope_cos, rope_sin, rope_dim / 2, pos_dev, n_head, n_kv,
                       eps);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_attn_decode(const float *q, uint64_t ldq, const float *kcache, const float *vcache,
                                const int *pos_dev, int ctx_bound, int B, int n_head, int n_kv, int head_dim,
                                float *out, uint64_t ldo)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (head_dim != ATT_HD) return QGPU_E_RANGE;
    if (!q || !kcache || !vcache || !pos_dev || !out || B < 1 || n_kv < 1 || n_head % n_kv || ctx_bound < B)
        return QGPU_E_ARG;
    if ((n_head / n_kv) * B > ATT_MAXQ) return QGPU_E_RANGE;
    const int nchunk = (ctx_bound + ATT_CS - 1) / ATT_CS;
    const size_t need = (size_t)n_kv * nchunk * ATT_MAXQ * (2 + ATT_HD) * sizeof(float);
    if (need > qg::ws_attn_bytes) {
        if (qg::ws_attn) {
            QG_CHECK(hipStreamSynchronize(qg::stream));
            QG_CHECK(hipFree(qg::ws_attn));
        }
        qg::ws_attn = nullptr;
        qg::ws_attn_bytes = 0;
        QG_CHECK(hipMalloc(&qg::ws_attn, need));
        qg::ws_attn_bytes = need;
    }
    float *pml = (float *)qg::ws_attn;
    float *po = pml + (size_t)n_kv * nchunk * ATT_MAXQ * 2;
    hipLaunchKernelGGL(k_attn_chunk, dim3(n_kv, nchunk), dim3(256), 0, qg::stream, q, ldq, kcache, vcache, pos_dev,
                       B, n_head, n_kv, nchunk, pml, po);
    QG_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head, B), dim3(ATT_HD), 0, qg::stream, q, ldq, pml, po, B, n_head,
                       n_kv, nchunk, out, ldo);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

// Reserve the attention workspace up front (so later calls never allocate,
// e.g. inside a captured graph): ctx_bound positions, n_kv heads.
extern "C" int qgpu_attn_reserve(int ctx_bound, int n_kv)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    const int nchunk = (ctx_bound + ATT_CS - 1) / ATT_CS;
    const size_t need = (size_t)n_kv * nchunk * ATT_MAXQ * (2 + ATT_HD) * sizeof(float);
    if (need <= qg::ws_attn_bytes) return QGPU_OK;
    if (qg::ws_attn) {
        QG_CHECK(hipStreamSynchronize(qg::stream));
        QG_CHECK(hipFree(qg::ws_attn));
        qg::ws_attn = nullptr;
    }
    QG_CHECK(hipMalloc(&qg::ws_attn, need));
    qg::ws_attn_bytes = need;
    return QGPU_OK;
}
