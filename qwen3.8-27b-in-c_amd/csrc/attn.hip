// Gated GQA decode attention for B query tokens (gfx950); reference
// model.c:318-406 (RoPE, per-head loop) and :760-810 (batched layer).
//
//  qgpu_attn_prep   : per-head RMSNorm of q and k, NeoX partial RoPE on the
//                     first rope_dim dims (pairs (i, i + rope_dim/2)), k and v
//                     written to the cache at position pos + b.
//  qgpu_attn_decode : softmax(q K^T / sqrt(hd)) V over positions t <= pos + b,
//                     times sigmoid(gate).  Flash-decoding: one block per
//                     (kv head, 64-position chunk) serves every query head of
//                     the group and every token of the batch (each K/V row is
//                     read once per chunk), then a combine pass merges chunks.
// Positions come from device memory (*pos_dev) so the launch sequence can be
// captured in a graph and replayed at any position.
#include "qgpu_internal.h"

#define ATT_HD   256
#define ATT_CS   64             // positions per chunk block
#define ATT_MAXQ 64             // row stride of the chunk partials
#define ATT_MAXR 48             // query rows (heads per kv head x batch) one chunk block serves

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

// Flash-decoding chunk kernel.  Block (g, c): kv head g, positions
// [c*ATT_CS, c*ATT_CS + ATT_CS), 8 waves.  Serves the QH = (n_head/n_kv) * B
// query rows of the group (row r = b * per + (h - g*per)); wave w owns rows
// w, w + 8, ... (<= ATT_RW of them).
//   FUSED = 1: the block also applies the per-head q/k RMSNorm and RoPE
//              (reference model.c:318-406): q rows are prepared in LDS (each
//              block recomputes them), the new k/v rows of positions pos..pos+B-1
//              that fall in this chunk are prepared here and written to the caches
//              (no other block reads them in this launch).
//   FUSED = 0: q rows already prepared, caches already hold every position.
// Every global load is issued first (K and V rows of the chunk, q rows).
// Scores: lane = position, K rows in LDS, q values broadcast from LDS, one
// running fp32 sum per row over d = 0..255.  Softmax statistics of a row are a
// reduction over the 64 lanes of one wave.  P.V: lane = 4 output dims, V rows
// (written over the K rows once the scores are done) and P from LDS.
// partials: pml [n_kv][nchunk][ATT_MAXQ][2] (m, l), po [n_kv][nchunk][ATT_MAXQ][ATT_HD]
#define ATT_KLD  260          // K row stride in LDS (floats)
#define ATT_NWV  8            // waves per chunk block
#define ATT_RW   (ATT_MAXR / ATT_NWV)

struct AttnArgs {
    const float *q; uint64_t ldq;
    const float *k, *v; uint64_t ldkv;
    const float *qw, *kw, *rcos, *rsin;
    float *kc, *vc;
    const int *pos_dev;
    float *pml, *po;
    int half, B, n_head, n_kv, nchunk;
    float eps;
};

static __device__ __forceinline__ float4 norm4(float4 v, float4 w, float sc)
{
    return make_float4((v.x * sc) * w.x, (v.y * sc) * w.y, (v.z * sc) * w.z, (v.w * sc) * w.w);
}

static __device__ __forceinline__ float wsum64(float v)
{
#pragma unroll
    for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

static __device__ __forceinline__ float wmax64(float v)
{
#pragma unroll
    for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// RW: rows per wave, ceil(QH / 8) (1..ATT_RW): the row loops carry no branches
template <int FUSED, int RW>
__global__ __launch_bounds__(ATT_NWV * 64) void k_attn_chunk(const AttnArgs p)
{
    __shared__ float Qs[ATT_MAXR][ATT_HD];       // first: its reads fit the 16-bit LDS offset field
    __shared__ float Ps[ATT_MAXR][ATT_CS];
    __shared__ float KV[ATT_CS * ATT_KLD];        // K rows (stride ATT_KLD), then V rows (stride ATT_HD)
    const int g = blockIdx.x, c = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int per = p.n_head / p.n_kv, QH = per * p.B;
    const int pos0 = *p.pos_dev, tmax = pos0 + p.B - 1, t0 = c * ATT_CS;
    float *ml = p.pml + ((uint64_t)g * p.nchunk + c) * ATT_MAXQ * 2;
    float *o = p.po + ((uint64_t)g * p.nchunk + c) * ATT_MAXQ * ATT_HD;
    if (t0 > tmax) {                              // chunk beyond the context: empty partial
        for (int qi = tid; qi < QH; qi += ATT_NWV * 64) { ml[2 * qi] = -INFINITY; ml[2 * qi + 1] = 0.0f; }
        return;
    }
    const uint64_t kvrow = (uint64_t)p.n_kv * ATT_HD;
    const int nt = min(ATT_CS, tmax - t0 + 1);    // positions of this chunk that exist
    // ---- every global load first: K and V rows pp = wv + 8i (lane = float4), q rows r = wv + 8i
    float4 kr[ATT_CS / ATT_NWV], vr[ATT_CS / ATT_NWV], qr[RW];
#pragma unroll
    for (int i = 0; i < ATT_CS / ATT_NWV; i++) {
        const int pp = wv + ATT_NWV * i, t = t0 + pp;
        kr[i] = vr[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (pp < nt) {
            if (FUSED && t >= pos0) {             // new row: raw k/v of token t - pos0
                const uint64_t off = (uint64_t)(t - pos0) * p.ldkv + (uint64_t)g * ATT_HD + 4 * lane;
                kr[i] = *(const float4 *)(p.k + off);
                vr[i] = *(const float4 *)(p.v + off);
            } else {
                const uint64_t off = (uint64_t)t * kvrow + (uint64_t)g * ATT_HD + 4 * lane;
                kr[i] = *(const float4 *)(p.kc + off);
                vr[i] = *(const float4 *)(p.vc + off);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RW; i++) {
        const int r = wv + ATT_NWV * i;
        qr[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (r < QH) {
            const int b = r / per, h = g * per + r % per;
            qr[i] = *(const float4 *)(p.q + (uint64_t)b * p.ldq + (uint64_t)h * 2 * ATT_HD + 4 * lane);
        }
    }
    float4 qw = make_float4(1.0f, 1.0f, 1.0f, 1.0f), kw = qw;
    if (FUSED) {
        qw = *(const float4 *)(p.qw + 4 * lane);
        kw = *(const float4 *)(p.kw + 4 * lane);
    }
    // ---- to LDS (per-head RMSNorm of q and of the new k rows on the way)
#pragma unroll
    for (int i = 0; i < ATT_CS / ATT_NWV; i++) {
        const int pp = wv + ATT_NWV * i, t = t0 + pp;
        float4 kv = kr[i];
        if (FUSED && pp < nt && t >= pos0) {
            const float ss = wsum64(kv.x * kv.x + kv.y * kv.y + kv.z * kv.z + kv.w * kv.w);
            kv = norm4(kv, kw, 1.0f / sqrtf(ss / (float)ATT_HD + p.eps));
        }
        *(float4 *)&KV[pp * ATT_KLD + 4 * lane] = kv;
    }
#pragma unroll
    for (int i = 0; i < RW; i++) {                // rows r >= QH hold zeros (their results are not used)
        const int r = wv + ATT_NWV * i;
        float4 qv = qr[i];
        if (FUSED && r < QH) {
            const float ss = wsum64(qv.x * qv.x + qv.y * qv.y + qv.z * qv.z + qv.w * qv.w);
            qv = norm4(qv, qw, 1.0f / sqrtf(ss / (float)ATT_HD + p.eps));
        }
        *(float4 *)&Qs[r][4 * lane] = qv;
    }
    __syncthreads();
    if (FUSED) {
        // NeoX RoPE on (i, i + half) at position pos0 + b: q rows and the new k rows of this chunk
        for (int e = tid; e < (QH + p.B) * p.half; e += ATT_NWV * 64) {
            const int r = e / p.half, i = e % p.half;
            float *x;
            int t;
            if (r < QH) { x = Qs[r]; t = pos0 + r / per; }
            else {
                t = pos0 + (r - QH);
                if (t < t0 || t >= t0 + ATT_CS) continue;
                x = &KV[(t - t0) * ATT_KLD];
            }
            const float cs = p.rcos[(uint64_t)t * p.half + i], sn = p.rsin[(uint64_t)t * p.half + i];
            const float v0 = x[i], v1 = x[i + p.half];
            x[i] = v0 * cs - v1 * sn;
            x[i + p.half] = v0 * sn + v1 * cs;
        }
        __syncthreads();
        // the new rows go to the caches (no other block of this launch reads them)
        for (int e = tid; e < p.B * 64; e += ATT_NWV * 64) {
            const int b = e >> 6, d4 = e & 63, t = pos0 + b;
            if (t < t0 || t >= t0 + ATT_CS) continue;
            const uint64_t row = (uint64_t)t * kvrow + (uint64_t)g * ATT_HD + 4 * d4;
            *(float4 *)(p.kc + row) = *(const float4 *)&KV[(t - t0) * ATT_KLD + 4 * d4];
        }
#pragma unroll
        for (int i = 0; i < ATT_CS / ATT_NWV; i++) {
            const int pp = wv + ATT_NWV * i, t = t0 + pp;
            if (pp < nt && t >= pos0)
                *(float4 *)(p.vc + (uint64_t)t * kvrow + (uint64_t)g * ATT_HD + 4 * lane) = vr[i];
        }
    }
    // ---- scores of this wave's rows at position t0 + lane
    const float scale = 1.0f / sqrtf((float)ATT_HD);
    {
        float s[RW];
#pragma unroll
        for (int j = 0; j < RW; j++) s[j] = 0.0f;
        const float *krow = &KV[lane * ATT_KLD];
#pragma unroll 4
        for (int d4 = 0; d4 < ATT_HD / 4; d4++) {
            const float4 kq = *(const float4 *)(krow + 4 * d4);
            float4 qv[RW];
#pragma unroll
            for (int j = 0; j < RW; j++) qv[j] = *(const float4 *)&Qs[wv + ATT_NWV * j][4 * d4];
#pragma unroll
            for (int j = 0; j < RW; j++) {
                s[j] = fmaf(qv[j].x, kq.x, s[j]); s[j] = fmaf(qv[j].y, kq.y, s[j]);
                s[j] = fmaf(qv[j].z, kq.z, s[j]); s[j] = fmaf(qv[j].w, kq.w, s[j]);
            }
        }
        // ---- chunk softmax statistics: a row's 64 scores are the 64 lanes of the wave
        const int t = t0 + lane;
#pragma unroll
        for (int j = 0; j < RW; j++) {
            const int r = wv + ATT_NWV * j;
            if (r >= QH) break;                   // wave-uniform
            const float sv = (lane < nt && t <= pos0 + r / per) ? s[j] * scale : -INFINITY;
            const float m = wmax64(sv);
            const float pr = m > -INFINITY ? expf(sv - m) : 0.0f;
            const float sum = wsum64(pr);
            Ps[r][lane] = pr;
            if (lane == 0) { ml[2 * r] = m; ml[2 * r + 1] = sum; }
        }
    }
    __syncthreads();                              // scores done: the K rows may be overwritten
#pragma unroll
    for (int i = 0; i < ATT_CS / ATT_NWV; i++) {
        const int pp = wv + ATT_NWV * i;
        *(float4 *)&KV[pp * ATT_HD + 4 * lane] = vr[i];
    }
    __syncthreads();
    // ---- P.V: lane = output dims 4*lane .. 4*lane+3 of this wave's rows
    float4 acc[RW];
#pragma unroll
    for (int j = 0; j < RW; j++) acc[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // positions beyond nt have P = 0 and V rows of zeros
#pragma unroll 4
    for (int pp = 0; pp < ATT_CS; pp++) {
        const float4 vv = *(const float4 *)&KV[pp * ATT_HD + 4 * lane];
        float pr[RW];
#pragma unroll
        for (int j = 0; j < RW; j++) pr[j] = Ps[wv + ATT_NWV * j][pp];
#pragma unroll
        for (int j = 0; j < RW; j++) {
            acc[j].x = fmaf(pr[j], vv.x, acc[j].x); acc[j].y = fmaf(pr[j], vv.y, acc[j].y);
            acc[j].z = fmaf(pr[j], vv.z, acc[j].z); acc[j].w = fmaf(pr[j], vv.w, acc[j].w);
        }
    }
#pragma unroll
    for (int j = 0; j < RW; j++) {
        const int r = wv + ATT_NWV * j;
        if (r < QH) *(float4 *)(o + (uint64_t)r * ATT_HD + 4 * lane) = acc[j];
    }
}

// out[b][h*hd + d] = sum_c o_c exp(m_c - M) / sum_c l_c exp(m_c - M) * sigmoid(gate); chunks past
// the last position (m = -inf) are skipped by the bound taken from *pos_dev
__global__ __launch_bounds__(ATT_HD) void k_attn_combine(const float *q, uint64_t ldq, const float *pml,
                                                         const float *po, const int *pos_dev, int B, int n_head,
                                                         int n_kv, int nchunk, float *out, uint64_t ldo)
{
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int per = n_head / n_kv, g = h / per, qi = b * per + (h % per);
    const int nc = min(nchunk, (*pos_dev + B - 1) / ATT_CS + 1);
    const float *mlg = pml + (uint64_t)g * nchunk * ATT_MAXQ * 2 + 2 * qi;
    const float *pog = po + (uint64_t)g * nchunk * ATT_MAXQ * ATT_HD + (uint64_t)qi * ATT_HD + d;
    float m = -INFINITY;
#pragma unroll 8
    for (int c = 0; c < nc; c++) m = fmaxf(m, mlg[(uint64_t)c * ATT_MAXQ * 2]);
    float l = 0.0f, acc = 0.0f;
#pragma unroll 8
    for (int c = 0; c < nc; c++) {
        const float mc = mlg[(uint64_t)c * ATT_MAXQ * 2];
        const float f = mc > -INFINITY ? expf(mc - m) : 0.0f;
        l = fmaf(mlg[(uint64_t)c * ATT_MAXQ * 2 + 1], f, l);
        acc = fmaf(pog[(uint64_t)c * ATT_MAXQ * ATT_HD], f, acc);
    }
    const float gate = q[(uint64_t)b * ldq + (uint64_t)h * 2 * ATT_HD + ATT_HD + d];
    out[(uint64_t)b * ldo + (uint64_t)h * ATT_HD + d] = (acc / l) * (1.0f / (1.0f + expf(-gate)));
}

static int attn_ws(int ctx_bound, int n_kv, int *nchunk)
{
    *nchunk = (ctx_bound + ATT_CS - 1) / ATT_CS;
    const size_t need = (size_t)n_kv * *nchunk * ATT_MAXQ * (2 + ATT_HD) * sizeof(float);
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
    return QGPU_OK;
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

static int attn_launch(const AttnArgs &a0, int fused, int ctx_bound, float *out, uint64_t ldo)
{
    AttnArgs a = a0;
    int rc = attn_ws(ctx_bound, a.n_kv, &a.nchunk);
    if (rc) return rc;
    a.pml = (float *)qg::ws_attn;
    a.po = a.pml + (size_t)a.n_kv * a.nchunk * ATT_MAXQ * 2;
    const int rw = ((a.n_head / a.n_kv) * a.B + ATT_NWV - 1) / ATT_NWV;
    const dim3 grid(a.n_kv, a.nchunk), blk(ATT_NWV * 64);
#define ATT_GO(F_, R_) hipLaunchKernelGGL((k_attn_chunk<F_, R_>), grid, blk, 0, qg::stream, a)
#define ATT_RWS(F_) do { switch (rw) { case 1: ATT_GO(F_, 1); break; case 2: ATT_GO(F_, 2); break; \
                         case 3: ATT_GO(F_, 3); break; case 4: ATT_GO(F_, 4); break; case 5: ATT_GO(F_, 5); break; \
                         default: ATT_GO(F_, 6); break; } } while (0)
    if (fused) ATT_RWS(1); else ATT_RWS(0);
#undef ATT_RWS
#undef ATT_GO
    QG_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_attn_combine, dim3(a.n_head, a.B), dim3(ATT_HD), 0, qg::stream, a.q, a.ldq, a.pml, a.po,
                       a.pos_dev, a.B, a.n_head, a.n_kv, a.nchunk, out, ldo);
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
    if (!q || !kcache || !vcache || !pos_dev || !out || B < 1 || n_kv < 1 || n_head % n_kv || ctx_bound < B ||
        ldq % 4 || ((uintptr_t)q & 15) || ((uintptr_t)kcache & 15) || ((uintptr_t)vcache & 15))
        return QGPU_E_ARG;
    if ((n_head / n_kv) * B > ATT_MAXR) return QGPU_E_RANGE;
    AttnArgs a = {};
    a.q = q; a.ldq = ldq; a.kc = (float *)kcache; a.vc = (float *)vcache; a.pos_dev = pos_dev;
    a.B = B; a.n_head = n_head; a.n_kv = n_kv;
    return attn_launch(a, 0, ctx_bound, out, ldo);
}

extern "C" int qgpu_attn_fused(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                               const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                               const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev,
                               int ctx_bound, int B, int n_head, int n_kv, int head_dim, float eps, float *out,
                               uint64_t ldo)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (head_dim != ATT_HD) return QGPU_E_RANGE;
    if (!q || !k || !v || !q_norm_w || !k_norm_w || !kcache || !vcache || !rope_cos || !rope_sin || !pos_dev ||
        !out || B < 1 || n_kv < 1 || n_head % n_kv || rope_dim < 2 || rope_dim > ATT_HD || rope_dim % 2 ||
        ctx_bound < B || ldq % 4 || ldkv % 4 || ((uintptr_t)q & 15) || ((uintptr_t)k & 15) || ((uintptr_t)v & 15) ||
        ((uintptr_t)kcache & 15) || ((uintptr_t)vcache & 15) || ((uintptr_t)q_norm_w & 15) ||
        ((uintptr_t)k_norm_w & 15))
        return QGPU_E_ARG;
    if ((n_head / n_kv) * B > ATT_MAXR) return QGPU_E_RANGE;
    AttnArgs a = {};
    a.q = q; a.ldq = ldq; a.k = k; a.v = v; a.ldkv = ldkv; a.qw = q_norm_w; a.kw = k_norm_w;
    a.rcos = rope_cos; a.rsin = rope_sin; a.kc = kcache; a.vc = vcache; a.pos_dev = pos_dev;
    a.half = rope_dim / 2; a.B = B; a.n_head = n_head; a.n_kv = n_kv; a.eps = eps;
    return attn_launch(a, 1, ctx_bound, out, ldo);
}

// Reserve the attention workspace up front (so later calls never allocate,
// e.g. inside a captured graph): ctx_bound positions, n_kv heads.
extern "C" int qgpu_attn_reserve(int ctx_bound, int n_kv)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (ctx_bound < 1 || n_kv < 1) return QGPU_E_ARG;
    int nchunk;
    return attn_ws(ctx_bound, n_kv, &nchunk);
}
