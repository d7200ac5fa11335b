// Gated DeltaNet verify block (gfx950): causal conv1d + SiLU, per-k-head L2
// norm and the delta-rule recurrence over B tokens, with one state snapshot
// per token (reference model.c:494-615, 845-941).
//
// Recurrent state lives in a ring of `nslot` slots per layer: the current
// state is slot *cur, and the state after token b of a batch is written to
// slot (*cur + 1 + b) % nslot, never over the current one.  Rolling back to
// "state after token j" (reference model_rollback_to, model.c:1015-1031, a
// 152 MB copy) is setting *cur to (*cur + 1 + j) % nslot.
#include "qgpu_internal.h"

#define GDN_MAXB 8
#define GDN_HK   128          // head_k_dim = head_v_dim (= ssm state size)
#define GDN_RB   16           // state rows per block
#define GDN_MAXBA QGPU_MAX_KS // partial planes of the gate inputs

static __device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

// state rows after each token: written once, read only by a later launch (rollback or the next verify)
static __device__ __forceinline__ void store_state8(float *p, const float (&S)[8])
{
    st_stream4(p, S[0], S[1], S[2], S[3]);
    st_stream4(p + 4, S[4], S[5], S[6], S[7]);
}

// one thread per channel: 4-tap causal conv over the sliding window, SiLU, snapshots
__global__ __launch_bounds__(256) void k_gdn_conv(const float *__restrict__ x, uint64_t ldx, int B, int conv_dim,
                                                  const float *__restrict__ w, float *__restrict__ ring,
                                                  uint64_t stride, int nslot, const int *__restrict__ cur_dev,
                                                  float *__restrict__ y, uint64_t ldy)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= conv_dim) return;
    const int cur = *cur_dev;
    const float4 s0 = *(const float4 *)(ring + (uint64_t)cur * stride + (uint64_t)c * 4);
    const float4 wc = *(const float4 *)(w + (uint64_t)c * 4);
    float win[4 + GDN_MAXB];
    win[0] = s0.x; win[1] = s0.y; win[2] = s0.z; win[3] = s0.w;
#pragma unroll
    for (int b = 0; b < GDN_MAXB; b++) {
        if (b >= B) break;
        win[4 + b] = x[(uint64_t)b * ldx + c];
        const float a0 = win[b + 1], a1 = win[b + 2], a2 = win[b + 3], a3 = win[b + 4];
        const float acc = ((a0 * wc.x + a1 * wc.y) + a2 * wc.z) + a3 * wc.w;
        y[(uint64_t)b * ldy + c] = silu_f(acc);
        const int slot = (cur + 1 + b) % nslot;
        *(float4 *)(ring + (uint64_t)slot * stride + (uint64_t)c * 4) = make_float4(a0, a1, a2, a3);
    }
}

// sum over the 16 lanes of a row group (lanes 16r .. 16r+15 of the wave)
static __device__ __forceinline__ float sum16(float v)
{
#pragma unroll
    for (int o = 8; o; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// (rowsum16: the same row sum with DPP lane moves, qgpu_internal.h)

// block = 16 state rows of one v-head; thread (row r = tid/16, column chunk cc = tid%16, 8 columns)
__global__ __launch_bounds__(256) void k_gdn_recur(const float *__restrict__ xq, uint64_t ldq,
                                                   const float *__restrict__ beta_raw,
                                                   const float *__restrict__ alpha_raw, uint64_t ldba,
                                                   const float *__restrict__ dt_bias, const float *__restrict__ ssm_a,
                                                   float *__restrict__ ring, uint64_t stride, int nslot,
                                                   const int *__restrict__ cur_dev, int B, int n_k, int n_v,
                                                   float eps, float *__restrict__ out, uint64_t ldo)
{
    const int h = blockIdx.x / (GDN_HK / GDN_RB);
    const int rb = blockIdx.x % (GDN_HK / GDN_RB);
    const int tid = threadIdx.x, r = tid >> 4, cc = tid & 15;
    const int j = rb * GDN_RB + r;                   // state row (v index)
    const int kh = h % n_k;                          // tiled v-head -> k-head map (model.c:565)
    const int cur = *cur_dev;
    const uint64_t hoff = (uint64_t)h * GDN_HK * GDN_HK + (uint64_t)j * GDN_HK + cc * 8;
    const float *S0 = ring + (uint64_t)cur * stride + hoff;
    float S[8];
    {
        const float4 a = *(const float4 *)S0, b = *(const float4 *)(S0 + 4);
        S[0] = a.x; S[1] = a.y; S[2] = a.z; S[3] = a.w; S[4] = b.x; S[5] = b.y; S[6] = b.z; S[7] = b.w;
    }
    const float qscale = 1.0f / sqrtf((float)GDN_HK);
    const float ah = ssm_a[h], dtb = dt_bias[h];
    for (int b = 0; b < B; b++) {
        const float *xb = xq + (uint64_t)b * ldq;
        const float *qp = xb + kh * GDN_HK + cc * 8;
        const float *kp = xb + n_k * GDN_HK + kh * GDN_HK + cc * 8;
        float q[8], k[8];
        {
            const float4 q0 = *(const float4 *)qp, q1 = *(const float4 *)(qp + 4);
            const float4 k0 = *(const float4 *)kp, k1 = *(const float4 *)(kp + 4);
            q[0] = q0.x; q[1] = q0.y; q[2] = q0.z; q[3] = q0.w; q[4] = q1.x; q[5] = q1.y; q[6] = q1.z; q[7] = q1.w;
            k[0] = k0.x; k[1] = k0.y; k[2] = k0.z; k[3] = k0.w; k[4] = k1.x; k[5] = k1.y; k[6] = k1.z; k[7] = k1.w;
        }
        float qq = 0.0f, kk = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) { qq = fmaf(q[i], q[i], qq); kk = fmaf(k[i], k[i], kk); }
        qq = sum16(qq);
        kk = sum16(kk);
        const float qn = sqrtf(qq), kn = sqrtf(kk);
        const float qs = 1.0f / (qn > eps ? qn : eps), ks = 1.0f / (kn > eps ? kn : eps);   // l2norm (kernels.c:780-805)
        float kq = 0.0f, sk = 0.0f, sq = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            q[i] *= qs;
            k[i] *= ks;
            kq = fmaf(k[i], q[i], kq);
            sk = fmaf(S[i], k[i], sk);
            sq = fmaf(S[i], q[i], sq);
        }
        kq = sum16(kq);
        sk = sum16(sk);
        sq = sum16(sq);
        const float beta = 1.0f / (1.0f + expf(-beta_raw[(uint64_t)b * ldba + h]));
        const float araw = alpha_raw[(uint64_t)b * ldba + h] + dtb;
        const float sp = araw > 30.0f ? araw : log1pf(expf(araw));
        const float decay = expf(ah * sp);
        const float vj = xb[2 * n_k * GDN_HK + (uint64_t)h * GDN_HK + j];
        const float dj = (vj - decay * sk) * beta;
        if (cc == 0) out[(uint64_t)b * ldo + (uint64_t)h * GDN_HK + j] = (decay * sq + dj * kq) * qscale;
#pragma unroll
        for (int i = 0; i < 8; i++) S[i] = fmaf(dj, k[i], decay * S[i]);
        store_state8(ring + (uint64_t)((cur + 1 + b) % nslot) * stride + hoff, S);
    }
}

// Conv and recurrence in one launch.  Block (v-head h, rows rb*16..rb*16+15)
// first runs the 4-tap conv + SiLU of the channels it reads: the 128 q and 128
// k channels of k-head h % n_k (recomputed by every block of that k-head; the
// window is a few floats per channel) and its own 16 v channels, for all B
// tokens, into LDS.  Conv-state snapshots are written once per channel: q/k
// channels by the block (h < n_k, rb = 0), v channels by their own block.
// Every global load of the block (state rows, conv windows and inputs of all
// tokens, gates) is issued before the first use; the L2 norms and q.k of all
// tokens are computed before the (sequential) recurrence, which then needs two
// row sums per token.  The state is read from ring slot *cur and the state after
// token b is written to slot (*cur + 1 + b) % nslot.
// Factor form (fst, fout): the state after token b is dec_b S + d_b kn_b^T, so a
// call may keep, instead of B snapshots, its starting state (slot *cur) and per
// token the row coefficients d_b (one per state row), the normalised k of each
// k-head and the decay: fout = 1 writes those to factor buffer fst[1] ^ 1.  The
// next call reads the state from slot *cur - P (P = fst[0] tokens kept: the
// rollback point + 1) and applies the P updates first, bit for bit as the call
// that kept them did; with fout = 1 it writes that state to slot *cur as its own
// base.
__global__ __launch_bounds__(256) void k_gdn_fused(const float *__restrict__ x, uint64_t ldx, const float *__restrict__ cw,
                                                   float *__restrict__ cring, uint64_t cstride,
                                                   const float *__restrict__ beta_raw, const float *__restrict__ alpha_raw,
                                                   uint64_t ldba, int ba_planes, uint64_t ba_pstride,
                                                   const float *__restrict__ dt_bias,
                                                   const float *__restrict__ ssm_a, float *__restrict__ sring,
                                                   uint64_t sstride, int nslot, const int *__restrict__ cur_dev, int B,
                                                   int n_k, int n_v, float eps, float *__restrict__ out, uint64_t ldo,
                                                   float *__restrict__ fbuf, uint64_t fts, const int *__restrict__ fst,
                                                   int fout)
{
    __shared__ float Yq[GDN_MAXB][GDN_HK], Yk[GDN_MAXB][GDN_HK], Yv[GDN_MAXB][GDN_RB];
    __shared__ float Gbeta[GDN_MAXB], Gdec[GDN_MAXB], Gkq[GDN_MAXB];
    __shared__ float Pb[GDN_MAXBA][GDN_MAXB], Pa[GDN_MAXBA][GDN_MAXB];   // gate planes [plane][token]
    const int h = blockIdx.x / (GDN_HK / GDN_RB);
    const int rb = blockIdx.x % (GDN_HK / GDN_RB);
    const int tid = threadIdx.x;
    const int kh = h % n_k;                          // tiled v-head -> k-head map (model.c:565)
    const int cur = *cur_dev;
    const bool own_qk = h < n_k && rb == 0;
    // factor form: P tokens of the previous call are still to be applied to the state in slot
    // *cur - P (their factors in buffer par of fbuf); this call's factors go to buffer par ^ 1
    const int P = fst ? min(max(fst[0], 0), min(GDN_MAXB, nslot - 1)) : 0;
    const int par = fst ? (fst[1] & 1) : 0;
    const float *fold = fbuf ? fbuf + (uint64_t)par * GDN_MAXB * fts : nullptr;
    float *fnew = fbuf ? fbuf + (uint64_t)(par ^ 1) * GDN_MAXB * fts : nullptr;
    const uint64_t fo_k = (uint64_t)n_v * GDN_HK, fo_g = fo_k + (uint64_t)n_k * GDN_HK;   // kn, decay offsets
    // ---- loads: this thread's 8 state columns
    const int r = tid >> 4, cc = tid & 15;
    const int j = rb * GDN_RB + r;                   // state row (v index)
    const uint64_t hoff = (uint64_t)h * GDN_HK * GDN_HK + (uint64_t)j * GDN_HK + cc * 8;
    const float *S0 = sring + (uint64_t)((cur - P + nslot) % nslot) * sstride + hoff;
    const float4 sa = *(const float4 *)S0, sbv = *(const float4 *)(S0 + 4);
    float S[8] = { sa.x, sa.y, sa.z, sa.w, sbv.x, sbv.y, sbv.z, sbv.w };
    // (row coefficient, decay and normalised k columns of each kept token; all loads issued first)
    float rdj[GDN_MAXB], rdec[GDN_MAXB];
    float4 rk0[GDN_MAXB], rk1[GDN_MAXB];
    if (P > 0) {                                     // uniform
#pragma unroll
        for (int p = 0; p < GDN_MAXB; p++) {
            const float *fp = fold + (uint64_t)(p < P ? p : P - 1) * fts;
            rdj[p] = fp[(uint64_t)h * GDN_HK + j];
            rdec[p] = fp[fo_g + h];
            rk0[p] = *(const float4 *)(fp + fo_k + (uint64_t)kh * GDN_HK + cc * 8);
            rk1[p] = *(const float4 *)(fp + fo_k + (uint64_t)kh * GDN_HK + cc * 8 + 4);
        }
    }

    // ---- loads: conv channel A (q or k channel tid) and, for tid < 16, channel B (v channel)
    const int cA = tid < GDN_HK ? kh * GDN_HK + tid : n_k * GDN_HK + kh * GDN_HK + (tid - GDN_HK);
    const bool hasB = tid < GDN_RB;
    const int cB = 2 * n_k * GDN_HK + h * GDN_HK + rb * GDN_RB + (tid & (GDN_RB - 1));
    const float4 s0A = *(const float4 *)(cring + (uint64_t)cur * cstride + (uint64_t)cA * 4);
    const float4 wA = *(const float4 *)(cw + (uint64_t)cA * 4);
    float xA[GDN_MAXB], xB[GDN_MAXB];
#pragma unroll
    for (int b = 0; b < GDN_MAXB; b++) xA[b] = x[(uint64_t)(b < B ? b : B - 1) * ldx + cA];
    float4 s0B = make_float4(0, 0, 0, 0), wB = make_float4(0, 0, 0, 0);
    if (hasB) {
        s0B = *(const float4 *)(cring + (uint64_t)cur * cstride + (uint64_t)cB * 4);
        wB = *(const float4 *)(cw + (uint64_t)cB * 4);
#pragma unroll
        for (int b = 0; b < GDN_MAXB; b++) xB[b] = x[(uint64_t)(b < B ? b : B - 1) * ldx + cB];
    }
    // ---- loads: per-token gate inputs of this head, one (plane, token) per thread (into LDS; summed
    // after the first barrier)
    if (tid < ba_planes * B) {
        const int q = tid / B, t = tid - q * B;
        const uint64_t o = (uint64_t)q * ba_pstride + (uint64_t)t * ldba + h;
        Pb[q][t] = beta_raw[o];
        Pa[q][t] = alpha_raw[o];
    }
    const float ah = ssm_a[h], dtb = dt_bias[h];
    // ---- conv + SiLU, conv-state snapshots
    {
        float *dA = tid < GDN_HK ? &Yq[0][tid] : &Yk[0][tid - GDN_HK];
        float win[4 + GDN_MAXB];
        win[0] = s0A.x; win[1] = s0A.y; win[2] = s0A.z; win[3] = s0A.w;
#pragma unroll
        for (int b = 0; b < GDN_MAXB; b++) {
            if (b >= B) break;
            win[4 + b] = xA[b];
            const float a0 = win[b + 1], a1 = win[b + 2], a2 = win[b + 3], a3 = win[b + 4];
            dA[b * GDN_HK] = silu_f(((a0 * wA.x + a1 * wA.y) + a2 * wA.z) + a3 * wA.w);
            if (own_qk) {
                const int slot = (cur + 1 + b) % nslot;
                st_stream4(cring + (uint64_t)slot * cstride + (uint64_t)cA * 4, a0, a1, a2, a3);
            }
        }
    }
    if (hasB) {
        float win[4 + GDN_MAXB];
        win[0] = s0B.x; win[1] = s0B.y; win[2] = s0B.z; win[3] = s0B.w;
#pragma unroll
        for (int b = 0; b < GDN_MAXB; b++) {
            if (b >= B) break;
            win[4 + b] = xB[b];
            const float a0 = win[b + 1], a1 = win[b + 2], a2 = win[b + 3], a3 = win[b + 4];
            Yv[b][tid] = silu_f(((a0 * wB.x + a1 * wB.y) + a2 * wB.z) + a3 * wB.w);
            const int slot = (cur + 1 + b) % nslot;
            st_stream4(cring + (uint64_t)slot * cstride + (uint64_t)cB * 4, a0, a1, a2, a3);
        }
    }
    __syncthreads();
    // ---- gates: beta = sigmoid(b), decay = exp(a * softplus(alpha + dt_bias)) (model.c:572-575), the
    // gate inputs summed over their planes in plane order
    if (tid < B) {
        float braw = Pb[0][tid], araw = Pa[0][tid];
        for (int q = 1; q < ba_planes; q++) {
            braw += Pb[q][tid];
            araw += Pa[q][tid];
        }
        Gbeta[tid] = 1.0f / (1.0f + expf(-braw));
        const float av = araw + dtb;
        const float sp = av > 30.0f ? av : log1pf(expf(av));
        Gdec[tid] = expf(ah * sp);
        if (fout && rb == 0) fnew[(uint64_t)tid * fts + fo_g + h] = Gdec[tid];
    }
    // ---- L2 norms (kernels.c:780-805) and q.k of every token, off the recurrence's serial path:
    // row group b (16 lanes) of the block handles token b, normalises its q and k in LDS and
    // keeps k.q of the normalised vectors
    if (r < B) {
        const int b = r;
        const float4 q0 = *(const float4 *)&Yq[b][cc * 8], q1 = *(const float4 *)&Yq[b][cc * 8 + 4];
        const float4 k0 = *(const float4 *)&Yk[b][cc * 8], k1 = *(const float4 *)&Yk[b][cc * 8 + 4];
        float q[8] = { q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w };
        float k[8] = { k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w };
        float qq = 0.0f, kk = 0.0f, kq = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) { qq = fmaf(q[i], q[i], qq); kk = fmaf(k[i], k[i], kk); kq = fmaf(k[i], q[i], kq); }
        qq = rowsum16(qq);
        kk = rowsum16(kk);
        kq = rowsum16(kq);
        const float qn = sqrtf(qq), kn = sqrtf(kk);
        const float qs = 1.0f / (qn > eps ? qn : eps), ks = 1.0f / (kn > eps ? kn : eps);
#pragma unroll
        for (int i = 0; i < 8; i++) { q[i] *= qs; k[i] *= ks; }
        // every lane of the row group holds the same sums; all write the same values
        *(float4 *)&Yq[b][cc * 8] = make_float4(q[0], q[1], q[2], q[3]);
        *(float4 *)&Yq[b][cc * 8 + 4] = make_float4(q[4], q[5], q[6], q[7]);
        *(float4 *)&Yk[b][cc * 8] = make_float4(k[0], k[1], k[2], k[3]);
        *(float4 *)&Yk[b][cc * 8 + 4] = make_float4(k[4], k[5], k[6], k[7]);
        if (cc == 0) Gkq[b] = kq * qs * ks;
    }
    __syncthreads();
    // factor form: the normalised k of every token, once per k-head
    if (fout && own_qk)
        for (int e = tid; e < B * GDN_HK; e += 256)
            fnew[(uint64_t)(e >> 7) * fts + fo_k + (uint64_t)kh * GDN_HK + (e & (GDN_HK - 1))] = Yk[e >> 7][e & (GDN_HK - 1)];
    // ---- the previous call's kept tokens, applied as it applied them (their loads were issued first;
    // applied here, after the conv phase, they add no wait: measured at 8192 positions, k = 5 / 7 forced
    // acceptance +0.4 / +1.3% against snapshots, -0.6 / -0.2% when applied before the conv phase)
    if (P > 0) {                                     // uniform
#pragma unroll
        for (int p = 0; p < GDN_MAXB; p++) {
            if (p >= P) break;
            const float k[8] = { rk0[p].x, rk0[p].y, rk0[p].z, rk0[p].w, rk1[p].x, rk1[p].y, rk1[p].z, rk1[p].w };
#pragma unroll
            for (int i = 0; i < 8; i++) S[i] = fmaf(rdj[p], k[i], rdec[p] * S[i]);
        }
        if (fout) store_state8(sring + (uint64_t)cur * sstride + hoff, S);   // the base of this call's factors
    }
    // ---- delta-rule recurrence: o = (g S q + d (k.q)) / sqrt(128), S <- g S + d k^T (model.c:494-615)
    const float qscale = 1.0f / sqrtf((float)GDN_HK);
#pragma unroll
    for (int b = 0; b < GDN_MAXB; b++) {
        if (b >= B) break;
        const float4 q0 = *(const float4 *)&Yq[b][cc * 8], q1 = *(const float4 *)&Yq[b][cc * 8 + 4];
        const float4 k0 = *(const float4 *)&Yk[b][cc * 8], k1 = *(const float4 *)&Yk[b][cc * 8 + 4];
        const float q[8] = { q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w };
        const float k[8] = { k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w };
        float sk = 0.0f, sq = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sk = fmaf(S[i], k[i], sk);
            sq = fmaf(S[i], q[i], sq);
        }
        sk = rowsum16(sk);
        sq = rowsum16(sq);
        const float beta = Gbeta[b], decay = Gdec[b], kq = Gkq[b];
        const float vj = Yv[b][r];
        const float dj = (vj - decay * sk) * beta;
        if (cc == 0) out[(uint64_t)b * ldo + (uint64_t)h * GDN_HK + j] = (decay * sq + dj * kq) * qscale;
#pragma unroll
        for (int i = 0; i < 8; i++) S[i] = fmaf(dj, k[i], decay * S[i]);
        if (fout) {
            if (cc == 0) fnew[(uint64_t)b * fts + (uint64_t)h * GDN_HK + j] = dj;
        } else {
            store_state8(sring + (uint64_t)((cur + 1 + b) % nslot) * sstride + hoff, S);
        }
    }
}

// The state after the P kept tokens of the last factor-form call, written to slot *cur (the
// base slot *cur - P plus the P rank-1 updates, in the order that call applied them).  Block
// (v-head, 16 rows), thread = (row, 8 columns), as k_gdn_fused.
__global__ __launch_bounds__(256) void k_gdn_materialize(float *__restrict__ sring, uint64_t sstride, int nslot,
                                                         const int *__restrict__ cur_dev,
                                                         const float *__restrict__ fbuf, uint64_t fts,
                                                         const int *__restrict__ fst, int n_k, int n_v)
{
    const int h = blockIdx.x / (GDN_HK / GDN_RB), rb = blockIdx.x % (GDN_HK / GDN_RB);
    const int tid = threadIdx.x, r = tid >> 4, cc = tid & 15, j = rb * GDN_RB + r, kh = h % n_k;
    const int cur = *cur_dev;
    const int P = min(max(fst[0], 0), min(GDN_MAXB, nslot - 1));
    if (P == 0) return;
    const float *fold = fbuf + (uint64_t)(fst[1] & 1) * GDN_MAXB * fts;
    const uint64_t fo_k = (uint64_t)n_v * GDN_HK, fo_g = fo_k + (uint64_t)n_k * GDN_HK;
    const uint64_t hoff = (uint64_t)h * GDN_HK * GDN_HK + (uint64_t)j * GDN_HK + cc * 8;
    const float *S0 = sring + (uint64_t)((cur - P + nslot) % nslot) * sstride + hoff;
    const float4 a = *(const float4 *)S0, c = *(const float4 *)(S0 + 4);
    float S[8] = { a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w };
    for (int p = 0; p < P; p++) {
        const float *fp = fold + (uint64_t)p * fts;
        const float dj = fp[(uint64_t)h * GDN_HK + j], dec = fp[fo_g + h];
        const float4 k0 = *(const float4 *)(fp + fo_k + (uint64_t)kh * GDN_HK + cc * 8);
        const float4 k1 = *(const float4 *)(fp + fo_k + (uint64_t)kh * GDN_HK + cc * 8 + 4);
        const float k[8] = { k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w };
#pragma unroll
        for (int i = 0; i < 8; i++) S[i] = fmaf(dj, k[i], dec * S[i]);
    }
    store_state8(sring + (uint64_t)cur * sstride + hoff, S);
}

// out[r] = rmsnorm(x[r], w) * silu(z[r]) for rows of n (per-head gated norm, model.c:928-941)
__global__ __launch_bounds__(128) void k_rmsnorm_gated(float *out, const float *x, const float *z, const float *w,
                                                       int n, uint64_t ld, float eps)
{
    __shared__ float sh[4];
    const float *xr = x + (uint64_t)blockIdx.x * ld;
    const float *zr = z + (uint64_t)blockIdx.x * ld;
    float *orow = out + (uint64_t)blockIdx.x * ld;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s = fmaf(xr[i], xr[i], s);
#pragma unroll
    for (int o = 32; o; o >>= 1) s += __shfl_xor(s, o);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    s = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += sh[i];
    const float scale = 1.0f / sqrtf(s / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) orow[i] = ((xr[i] * scale) * w[i]) * silu_f(zr[i]);
}

extern "C" int qgpu_gdn_conv(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w, float *ring,
                             uint64_t slot_stride, int nslot, const int *cur, float *y, uint64_t ldy)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!x || !conv_w || !ring || !cur || !y || B < 1 || B > GDN_MAXB || nslot < B + 1 || conv_dim < 1 ||
        slot_stride < (uint64_t)conv_dim * 4 || ldx < (uint64_t)conv_dim || ldy < (uint64_t)conv_dim)
        return QGPU_E_ARG;
    hipLaunchKernelGGL(k_gdn_conv, dim3((conv_dim + 255) / 256), dim3(256), 0, qg::stream, x, ldx, B, conv_dim,
                       conv_w, ring, slot_stride, nslot, cur, y, ldy);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_gdn_recurrence(const float *xq, uint64_t ldq, const float *beta_raw, const float *alpha_raw,
                                   uint64_t ldba, const float *dt_bias, const float *ssm_a, float *ring,
                                   uint64_t slot_stride, int nslot, const int *cur, int B, int n_k, int n_v,
                                   int head_dim, float eps, float *out, uint64_t ldo)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (head_dim != GDN_HK) return QGPU_E_RANGE;
    if (!xq || !beta_raw || !alpha_raw || !dt_bias || !ssm_a || !ring || !cur || !out || B < 1 || B > GDN_MAXB ||
        nslot < B + 1 || n_k < 1 || n_v < 1 || slot_stride < (uint64_t)n_v * GDN_HK * GDN_HK ||
        ldq < (uint64_t)(2 * n_k + n_v) * GDN_HK || ldo < (uint64_t)n_v * GDN_HK || ldba < (uint64_t)n_v)
        return QGPU_E_ARG;
    hipLaunchKernelGGL(k_gdn_recur, dim3(n_v * (GDN_HK / GDN_RB)), dim3(256), 0, qg::stream, xq, ldq, beta_raw,
                       alpha_raw, ldba, dt_bias, ssm_a, ring, slot_stride, nslot, cur, B, n_k, n_v, eps, out, ldo);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_rmsnorm_gated(float *out, const float *x, const float *z, const float *w, int n, int rows,
                                  uint64_t ld, float eps)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!out || !x || !z || !w || n < 1 || rows < 0 || ld < (uint64_t)n) return QGPU_E_ARG;
    if (!rows) return QGPU_OK;
    hipLaunchKernelGGL(k_rmsnorm_gated, dim3(rows), dim3(128), 0, qg::stream, out, x, z, w, n, ld, eps);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_gdn_fused_factor(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w,
                                     float *conv_ring, uint64_t conv_stride, const float *beta_raw,
                                     const float *alpha_raw, uint64_t ldba, int ba_planes, uint64_t ba_pstride,
                                     const float *dt_bias, const float *ssm_a, float *ssm_ring, uint64_t ssm_stride,
                                     int nslot, const int *cur, int n_k, int n_v, int head_dim, float eps, float *out,
                                     uint64_t ldo, float *factors, uint64_t f_tok, const int *fstate, int factor_out)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (head_dim != GDN_HK) return QGPU_E_RANGE;
    if ((fstate || factor_out) &&
        (!factors || ((uintptr_t)factors & 15) || f_tok % 4 || f_tok < (uint64_t)(n_v + n_k) * GDN_HK + n_v))
        return QGPU_E_ARG;
    if (!x || !conv_w || !conv_ring || !beta_raw || !alpha_raw || !dt_bias || !ssm_a || !ssm_ring || !cur || !out ||
        B < 1 || B > GDN_MAXB || nslot < B + 1 || n_k < 1 || n_v < 1 ||
        conv_dim != (2 * n_k + n_v) * GDN_HK || conv_stride < (uint64_t)conv_dim * 4 ||
        ssm_stride < (uint64_t)n_v * GDN_HK * GDN_HK || ldx < (uint64_t)conv_dim || ldo < (uint64_t)n_v * GDN_HK ||
        ldba < (uint64_t)n_v || ((uintptr_t)conv_ring & 15) || ((uintptr_t)conv_w & 15) || ((uintptr_t)ssm_ring & 15) ||
        conv_stride % 4 || ssm_stride % 4 || ba_planes < 1 || ba_planes > GDN_MAXBA || ba_planes * B > 256 ||
        (ba_planes > 1 && ba_pstride < (uint64_t)B * ldba))
        return QGPU_E_ARG;
    hipLaunchKernelGGL(k_gdn_fused, dim3(n_v * (GDN_HK / GDN_RB)), dim3(256), 0, qg::stream, x, ldx, conv_w, conv_ring,
                       conv_stride, beta_raw, alpha_raw, ldba, ba_planes, ba_pstride, dt_bias, ssm_a, ssm_ring,
                       ssm_stride, nslot, cur, B, n_k, n_v, eps, out, ldo, factors, f_tok, fstate, factor_out ? 1 : 0);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_gdn_fused_planes(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w,
                                     float *conv_ring, uint64_t conv_stride, const float *beta_raw,
                                     const float *alpha_raw, uint64_t ldba, int ba_planes, uint64_t ba_pstride,
                                     const float *dt_bias, const float *ssm_a, float *ssm_ring, uint64_t ssm_stride,
                                     int nslot, const int *cur, int n_k, int n_v, int head_dim, float eps, float *out,
                                     uint64_t ldo)
{
    return qgpu_gdn_fused_factor(x, ldx, B, conv_dim, conv_w, conv_ring, conv_stride, beta_raw, alpha_raw, ldba,
                                 ba_planes, ba_pstride, dt_bias, ssm_a, ssm_ring, ssm_stride, nslot, cur, n_k, n_v,
                                 head_dim, eps, out, ldo, nullptr, 0, nullptr, 0);
}

extern "C" int qgpu_gdn_materialize(float *ssm_ring, uint64_t ssm_stride, int nslot, const int *cur, int n_k, int n_v,
                                    int head_dim, const float *factors, uint64_t f_tok, const int *fstate)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (head_dim != GDN_HK) return QGPU_E_RANGE;
    if (!ssm_ring || !cur || !factors || !fstate || n_k < 1 || n_v < 1 || nslot < 2 ||
        ssm_stride < (uint64_t)n_v * GDN_HK * GDN_HK || ((uintptr_t)ssm_ring & 15) || ssm_stride % 4 ||
        ((uintptr_t)factors & 15) || f_tok % 4 || f_tok < (uint64_t)(n_v + n_k) * GDN_HK + n_v)
        return QGPU_E_ARG;
    hipLaunchKernelGGL(k_gdn_materialize, dim3(n_v * (GDN_HK / GDN_RB)), dim3(256), 0, qg::stream, ssm_ring, ssm_stride,
                       nslot, cur, factors, f_tok, fstate, n_k, n_v);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_gdn_fused(const float *x, uint64_t ldx, int B, int conv_dim, const float *conv_w, float *conv_ring,
                              uint64_t conv_stride, const float *beta_raw, const float *alpha_raw, uint64_t ldba,
                              const float *dt_bias, const float *ssm_a, float *ssm_ring, uint64_t ssm_stride, int nslot,
                              const int *cur, int n_k, int n_v, int head_dim, float eps, float *out, uint64_t ldo)
{
    return qgpu_gdn_fused_planes(x, ldx, B, conv_dim, conv_w, conv_ring, conv_stride, beta_raw, alpha_raw, ldba, 1, 0,
                                 dt_bias, ssm_a, ssm_ring, ssm_stride, nslot, cur, n_k, n_v, head_dim, eps, out, ldo);
}

