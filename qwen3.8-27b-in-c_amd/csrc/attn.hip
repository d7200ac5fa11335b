// Gated GQA decode attention for B query tokens (gfx950); reference
// model.c:318-406 (RoPE, per-head loop) and :760-810 (batched layer).
//
//  qgpu_attn_prep   : per-head RMSNorm of q and k, NeoX partial RoPE on the
//                     first rope_dim dims (pairs (i, i + rope_dim/2)), k and v
//                     written to the cache at position pos + b.
//  qgpu_attn_decode : softmax(q K^T / sqrt(hd)) V over positions t <= pos + b,
//                     times sigmoid(gate).  Flash-decoding on the matrix cores:
//                     one block per (kv head, span of 16-position tiles) serves
//                     every query head of the group and every token of the batch
//                     (each K/V row is read once per launch), then a combine pass
//                     merges the spans.
// Positions come from device memory (*pos_dev) so the launch sequence can be
// captured in a graph and replayed at any position.
#include "qgpu_internal.h"
#include <climits>

#define ATT_HD   256
#define ATT_MAXQ 64             // row stride of the span partials
#define ATT_MAXR 48             // query rows (heads per kv head x batch) one span block serves

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

// Span kernel (flash decoding on the matrix cores).  Block (g, s): kv head g,
// span s of 16-position tiles, NW waves; wave w owns head dims [DW w, DW w + DW),
// DW = 256 / NW (NW = 8, DW = 32 in every launch).
// It serves every query row of the group, r = b * per + (h - g*per) < QH =
// per * B, as NRT row tiles of 16.
//   * Scores, per tile and row tile: S^T (16 positions x 16 rows) = K Q^T as three
//     fp16 split products (hi hi + hi lo + lo hi, v_mfma_f32_16x16x32_f16), lane l
//     supplying K[pos l%16][d] and Q[row l%16][d] for its 8 dims d = DW w + 16q +
//     4(l/16) + j, q < 2, j < 4 (any order of the d sum is the same dot product).
//     Each wave writes its partial tile to LDS.
//   * Softmax: the rows are cut into units of 4 (16 positions each: one value per
//     lane); the wave that owns a unit sums the NW partial scores in wave order,
//     keeps the running max and sum of its rows (scores in log2 units, exp2), and
//     writes the probabilities and the rows' rescale factors to LDS.
//   * P.V: the probabilities come back as bf16 hi and lo parts in the score
//     accumulator's layout (lane l: positions 4(l/16) .. 4(l/16) + 3, row l%16), the
//     A operand of a 16-position product (three bf16 split products,
//     v_mfma_f32_16x16x16_bf16); lane l supplies V[those positions][DW w + NQ (l%16)
//     + c] for output tile c.  O accumulates in fp32 registers (lane l, register r:
//     row 4(l/16) + r).
//   * Step t: loads of tile t + 2, the softmax of tile t beside the scores of tile
//     t + 1, one barrier, P.V of tile t (a ring of three K/V register slots).
//   FUSED = 1: the block also applies the per-head q/k RMSNorm and RoPE
//              (reference model.c:318-406) in LDS: q rows, and the new k rows
//              of positions pos..pos+B-1; the new k and v rows replace the
//              cached rows of those positions when a tile is used, and the block
//              whose span holds a new position writes them to the caches (no
//              block reads new rows from the caches in this launch).
//   FUSED = 0: q rows already prepared, caches already hold every position.
// The number of spans follows the live context: ntl tiles hold positions
// 0..pos+B-1; nsl = ceil(ntl / tps) spans of tps tiles, for at most nspan
// spans (the launch size); blocks past nsl exit and the combine skips them.
// partials: pml [n_kv][nspan][ATT_MAXQ][2] (m, l), po [n_kv][nspan][ATT_MAXQ][ATT_HD]; m is the
// running maximum of the scores in log2 units (q.k / sqrt(hd) * log2 e), l = sum of exp2(s - m)
#define ATT_TP    16          // positions per tile
#define ATT_MAXB  8           // new positions per fused call
#ifndef ATT_NSPAN
#define ATT_NSPAN 64          // spans per kv head at most
#endif
#define ATT_RECORDS 0x7FFFFFFFu   // bytes the K/V buffer resources cover (offsets are < 2^31)
#define ATT_OOB 0x80000000u       // an offset at or past ATT_RECORDS: the load reads zeros, fetches nothing
static_assert(ATT_OOB >= ATT_RECORDS, "dead K/V loads must fall outside the buffer resource");
#ifndef ATT_NW3
#define ATT_NW3 8             // waves of the three-row-tile span kernel
#endif
#ifndef ATT_MINTPS
#define ATT_MINTPS 2          // tiles per span at least (800 positions, B = 4 / 8: 15.4 / 20.2 -> 14.4 / 17.8 us
                              // per call against 1; 4: 15.2 / 18.7 us)
#endif

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
template <int N> struct VSlice;                     // a lane's V slice of N dims
template <> struct VSlice<4> { typedef v4f T; };
template <> struct VSlice<2> { typedef v2f T; };

struct AttnArgs {
    const float *q; uint64_t ldq;
    const float *k, *v; uint64_t ldkv;
    const float *qw, *kw, *rcos, *rsin;
    float *kc, *vc;
    const int *pos_dev;
    float *pml, *po;
    int half, B, n_head, n_kv, nspan;
    float eps;
};

// live tiles ntl, tiles per span tps and spans with work nsl, from the device
// position (the span kernel and the combine derive the same split)
static __host__ __device__ __forceinline__ void span_split(int pos0, int B, int nspan, int &ntl, int &tps, int &nsl)
{
    ntl = (pos0 + B + ATT_TP - 1) / ATT_TP;
    const int ns = ntl < nspan ? ntl : nspan;
    tps = (ntl + ns - 1) / ns;
    if (tps < ATT_MINTPS) tps = ATT_MINTPS;
    nsl = (ntl + tps - 1) / tps;
}

// Split-precision products on the half-precision matrix cores.  An fp32 operand x is held as
// hi + lo, hi = x rounded to the narrow type, lo = (x - hi) rounded (x - hi is exact in fp32);
// a product a b is summed as a_hi b_hi + a_hi b_lo + a_lo b_hi in fp32 accumulators (the
// dropped a_lo b_lo and the two roundings are below 2^-2p relative for a p-bit significand).
//   fp16 (p = 11): |x - hi - lo| <= 2^-22 |x|, range |x| < 65504: the q and k rows, which are
//                  RMS-normalised (|x| <= sqrt(head_dim) * |norm weight|);
//   bf16 (p = 8):  2^-16 |x|, the fp32 range: the probabilities and the v rows (unbounded).
// v_mfma_f32_16x16x32_f16 does 16 x 16 x 32 multiply-adds in 16 cycles and
// v_mfma_f32_16x16x16_bf16 16 x 16 x 16 in 8, against 16 x 16 x 4 in 32 for the fp32 form: the
// three products cost 5.3x fewer matrix-core cycles than one fp32 product.
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 v4b __attribute__((ext_vector_type(4)));
struct SplitH { v8h hi, lo; };
struct SplitB { v4s hi, lo; };
// two values: one packed convert for hi, its two halves widened back exactly, one packed convert
// of the differences for lo: 6 instructions per pair
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
static __device__ __forceinline__ void split_h2(float x0, float x1, v2h &hi, v2h &lo)
{
    hi = __builtin_convertvector((v2f{x0, x1}), v2h);
    const v2f w = __builtin_convertvector(hi, v2f);
    lo = __builtin_convertvector((v2f{x0 - w[0], x1 - w[1]}), v2h);
}
static __device__ __forceinline__ SplitH split_h8(v4f x0, v4f x1)
{
    SplitH r;
    v2h h[4], l[4];
    split_h2(x0[0], x0[1], h[0], l[0]);
    split_h2(x0[2], x0[3], h[1], l[1]);
    split_h2(x1[0], x1[1], h[2], l[2]);
    split_h2(x1[2], x1[3], h[3], l[3]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r.hi[2 * i] = h[i][0]; r.hi[2 * i + 1] = h[i][1];
        r.lo[2 * i] = l[i][0]; r.lo[2 * i + 1] = l[i][1];
    }
    return r;
}
// two values: hi = the pair rounded to bf16 (one packed convert), widened back exactly by a shift
// and a mask, lo = the rounded differences (one packed convert): 6 instructions per pair
typedef __bf16 v2b __attribute__((ext_vector_type(2)));
static __device__ __forceinline__ void split_b2(float x0, float x1, uint32_t &hi, uint32_t &lo)
{
    v2f x = {x0, x1};
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2b));
    const float d0 = x0 - __builtin_bit_cast(float, hi << 16), d1 = x1 - __builtin_bit_cast(float, hi & 0xFFFF0000u);
    v2f d = {d0, d1};
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(d, v2b));
}
static __device__ __forceinline__ SplitB split_b4(float x0, float x1, float x2, float x3)
{
    uint32_t h0, l0, h1, l1;
    split_b2(x0, x1, h0, l0);
    split_b2(x2, x3, h1, l1);
    return SplitB{ __builtin_bit_cast(v4s, make_uint2(h0, h1)), __builtin_bit_cast(v4s, make_uint2(l0, l1)) };
}
static __device__ __forceinline__ v4f mfma_split_h(const SplitH &a, const SplitH &b, v4f c)
{
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.lo, b.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.hi, b.lo, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.hi, b.hi, c, 0, 0, 0);
}
static __device__ __forceinline__ v4f mfma_split_b(const SplitB &a, const SplitB &b, v4f c)
{
    c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.lo, b.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.hi, b.lo, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.hi, b.hi, c, 0, 0, 0);
}

template <int FUSED, int NRT, int ATT_NWV, int HS>
__global__ __launch_bounds__(ATT_NWV * 64) void k_attn_span(const AttnArgs p)
{
    static_assert(HS == 1 || HS == 2, "one block or two per (kv head, span)");
    constexpr int ATT_DW = ATT_HD / ATT_NWV;      // head dims per wave
    constexpr int ATT_NQ = ATT_DW / 16;           // float4 operand loads per row and 16-dim output tiles per wave
    typedef typename VSlice<ATT_NQ>::T vqf;
    // score exchange: per (buffer, wave, row tile) the 64 lanes' v4f, one 16-byte pad after every 16
    // lanes (68 slots), so the 16 lanes of a softmax row (4 lane groups, same n) read distinct banks
    constexpr int SXS = 68;                                        // v4f slots per (buffer, wave, row tile)
    constexpr int SXF = 2 * ATT_NWV * NRT * SXS * 4;               // floats of the score exchange
    __shared__ float lds[FUSED && NRT * 16 * ATT_HD > SXF ? NRT * 16 * ATT_HD : SXF];   // q rows (FUSED), then the score exchange
    __shared__ float Kn[FUSED ? ATT_MAXB : 1][ATT_HD];   // new k rows, normalised and rotated
    __shared__ float Vn[FUSED ? ATT_MAXB : 1][ATT_HD];   // new v rows
    __shared__ float Rc[FUSED ? ATT_MAXB * ATT_HD / 2 : 1], Rs[FUSED ? ATT_MAXB * ATT_HD / 2 : 1];   // RoPE tables
    // probabilities [buf][rt][gq][n][v] as bf16 hi and lo parts: the softmax owner splits each once; the
    // P.V lanes read their four positions' parts with one 8-byte load each
    __shared__ __attribute__((aligned(16))) uint16_t Ph[2 * NRT * 256], Plo[2 * NRT * 256];
    __shared__ __attribute__((aligned(16))) float Al[2 * NRT * 16];    // rescale factors [buf][row]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, gq = lane >> 4;
    // HS = 2: the query heads of a kv head are split between two blocks, halves hh = 0, 1, each
    // serving per / 2 heads of every token.  Blocks L and L + 8 (one XCD under round-robin dispatch,
    // so the second finds the K/V rows in the same L2) take the two halves of one (kv head, span)
    // pair u, pairs in span order (the blocks of spans with work come first).
    int g, s, hh = 0;
    if (HS == 1) {
        g = blockIdx.x;
        s = blockIdx.y;
    } else {
        const int L = blockIdx.x, q8 = L >> 3, u = (q8 >> 1) * 8 + (L & 7);
        hh = q8 & 1;
        if (u >= p.n_kv * p.nspan) return;
        g = u % p.n_kv;
        s = u / p.n_kv;
    }
    const int per = p.n_head / p.n_kv, pr = per / HS, QH = pr * p.B;
    // r / pr for the row indices 0 <= r < 64 of this kernel: (r * ceil(2^16 / pr)) >> 16 is exact there
    // (the rounding up adds less than r / 2^16 < 1 / pr to r / pr)
    const uint32_t inv_per = (65536u + (uint32_t)pr - 1u) / (uint32_t)pr;
    auto divp = [&](int r) { return (int)(((uint32_t)r * inv_per) >> 16); };
    // block row r (token b = r / pr, head j = r - b pr of the block's) is row b per + hh pr + j of
    // the kv head's partials and query head g per + hh pr + j
    auto rfull = [&](int r) { return HS == 1 ? r : r + divp(r) * (per - pr) + hh * pr; };
    const uint64_t kvrow = (uint64_t)p.n_kv * ATT_HD, hoff = (uint64_t)g * ATT_HD;
    const int d0 = ATT_DW * wv;

    // ---- loads that do not depend on the position first: q rows (FUSED: raw rows for the
    // prologue; else the Q operands, row rt*16 + n, dims d0 + 16q + 4gq .. +3), the new k
    // rows and the norm weights
    constexpr int QV = FUSED ? NRT * 16 * 64 / (ATT_NWV * 64) : 1;   // float4 of q rows per thread
    constexpr int KV = FUSED ? ATT_MAXB * 64 / (ATT_NWV * 64) : 1;
    float4 qv[QV], knv[KV], vnv[KV], qw = make_float4(0.0f, 0.0f, 0.0f, 0.0f), kw = qw;
    v4f qop[NRT][ATT_NQ];
    if (FUSED) {
#pragma unroll
        for (int u = 0; u < QV; u++) {
            const int e = tid + u * ATT_NWV * 64, r = e >> 6, d4 = e & 63;
            qv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (r < QH) {
                const int b = divp(r), h = g * per + hh * pr + (r - b * pr);
                qv[u] = *(const float4 *)(p.q + (uint64_t)b * p.ldq + (uint64_t)h * 2 * ATT_HD + 4 * d4);
            }
        }
#pragma unroll
        for (int u = 0; u < KV; u++) {
            const int e = tid + u * ATT_NWV * 64, b = e >> 6, d4 = e & 63;
            knv[u] = vnv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (b < p.B) {
                knv[u] = *(const float4 *)(p.k + (uint64_t)b * p.ldkv + hoff + 4 * d4);
                vnv[u] = *(const float4 *)(p.v + (uint64_t)b * p.ldkv + hoff + 4 * d4);
            }
        }
        qw = *(const float4 *)(p.qw + 4 * lane);
        kw = *(const float4 *)(p.kw + 4 * lane);
    } else {
#pragma unroll
        for (int rt = 0; rt < NRT; rt++) {
            const int r = rt * 16 + n;
            const int b = divp(r), h = g * per + hh * pr + (r - b * pr);
#pragma unroll
            for (int q = 0; q < ATT_NQ; q++)
                qop[rt][q] = r < QH ? *(const v4f *)(p.q + (uint64_t)b * p.ldq + (uint64_t)h * 2 * ATT_HD + d0 + 16 * q + 4 * gq)
                                    : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    const int pos0 = *p.pos_dev, tmax = pos0 + p.B - 1;
    int ntl, tps, nsl;
    span_split(pos0, p.B, p.nspan, ntl, tps, nsl);
    if (s >= nsl) return;
    const int tile0 = s * tps, tile1 = min(tile0 + tps, ntl);
    const int posA = tile0 * ATT_TP, posB = min(tile1 * ATT_TP, tmax + 1);   // positions of this span

    // ---- operand loads of tile tt into a ring slot: the cached K and V rows through buffer loads
    // at 32-bit offsets from this kv head's row 0.  Rows past the live end read row tmax instead
    // (the mask gives them probability 0, and the row is finite).  FUSED: the rows of positions
    // pos0.. (not in the caches before this launch) are replaced from Kn and Vn when the tile is
    // used.  Every lane loads every tile, so the loads are straight-line code and the wait for a
    // slot counts exactly the loads issued after it.
    const __amdgpu_buffer_rsrc_t rsK = __builtin_amdgcn_make_buffer_rsrc((void *)(p.kc + hoff), 0, (int)ATT_RECORDS, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc((void *)(p.vc + hoff), 0, (int)ATT_RECORDS, 0x00020000);
    const uint32_t rowb = (uint32_t)kvrow * 4u;
    // a tile whose rows are all live: lane offsets of the tile's first row (computed once) plus the
    // tile's row offset in a scalar register; the last tile of the live context: clamped rows
    const uint32_t kofs = (uint32_t)n * rowb + (uint32_t)(d0 + 4 * gq) * 4u;
    uint32_t vofs[4];
#pragma unroll
    for (int v = 0; v < 4; v++) vofs[v] = (uint32_t)(4 * gq + v) * rowb + (uint32_t)(d0 + ATT_NQ * n) * 4u;
    // live = 0: the loads are issued (so every path issues the same loads) at an offset past the
    // buffer's end: they read zeros and fetch nothing
    auto load_kv = [&](int tt, v4f *kr_, vqf *vr_, bool live) {
        const int p0 = tt * ATT_TP;
        uint32_t ko = kofs, vo[4] = { vofs[0], vofs[1], vofs[2], vofs[3] }, so = (uint32_t)p0 * rowb;
        if (!live) {                               // wave-uniform
            ko = ATT_OOB;
#pragma unroll
            for (int v = 0; v < 4; v++) vo[v] = ATT_OOB;
            so = 0;
        } else if (p0 + ATT_TP - 1 > tmax) {      // wave-uniform
            ko = (uint32_t)min(p0 + n, tmax) * rowb + (uint32_t)(d0 + 4 * gq) * 4u;
#pragma unroll
            for (int v = 0; v < 4; v++)
                vo[v] = (uint32_t)min(p0 + 4 * gq + v, tmax) * rowb + (uint32_t)(d0 + ATT_NQ * n) * 4u;
            so = 0;
        }
#pragma unroll
        for (int q = 0; q < ATT_NQ; q++)
            kr_[q] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rsK, ko + 64u * q, so, 0));
#pragma unroll
        for (int v = 0; v < 4; v++) {
            if constexpr (ATT_NQ == 4)
                vr_[v] = __builtin_bit_cast(vqf, __builtin_amdgcn_raw_buffer_load_b128(rsV, vo[v], so, 0));
            else
                vr_[v] = __builtin_bit_cast(vqf, __builtin_amdgcn_raw_buffer_load_b64(rsV, vo[v], so, 0));
        }
    };
    // a ring of three operand slots: tile t sits in slot (t - tile0) % 3.  Its K is used one
    // step before its V (scores run a tile ahead of P.V), and its loads are issued two steps
    // before its V is used.  The first two tiles' loads are issued before the q preparation.
    constexpr int NSL = 3;
    v4f kr[NSL][ATT_NQ];
    vqf vr[NSL][4];
    // (loads are issued for every step, past the span's last tile too, as loads that fetch
    // nothing: every path then issues the same loads and the waits count them exactly)
    load_kv(tile0, kr[0], vr[0], true);
    load_kv(tile0 + 1, kr[1], vr[1], tile0 + 1 < tile1);

    if (FUSED) {
        float (*Qs)[ATT_HD] = (float (*)[ATT_HD])lds;
        const bool has_new = posB > pos0;
        float cv[ATT_MAXB * ATT_HD / 2 / (ATT_NWV * 64)], sv[ATT_MAXB * ATT_HD / 2 / (ATT_NWV * 64)];
#pragma unroll
        for (int u = 0; u < ATT_MAXB * ATT_HD / 2 / (ATT_NWV * 64); u++) {
            const int e = tid + u * ATT_NWV * 64, b = e / p.half, i = e % p.half;
            cv[u] = sv[u] = 0.0f;
            if (b < p.B) {
                cv[u] = p.rcos[(uint64_t)(pos0 + b) * p.half + i];
                sv[u] = p.rsin[(uint64_t)(pos0 + b) * p.half + i];
            }
        }
#pragma unroll
        for (int u = 0; u < QV; u++) {
            const int e = tid + u * ATT_NWV * 64;
            *(float4 *)&Qs[e >> 6][4 * (e & 63)] = qv[u];
        }
#pragma unroll
        for (int u = 0; u < KV; u++) {
            const int e = tid + u * ATT_NWV * 64;
            *(float4 *)&Kn[e >> 6][4 * (e & 63)] = knv[u];
            *(float4 *)&Vn[e >> 6][4 * (e & 63)] = vnv[u];
        }
#pragma unroll
        for (int u = 0; u < ATT_MAXB * ATT_HD / 2 / (ATT_NWV * 64); u++) {
            const int e = tid + u * ATT_NWV * 64;
            Rc[e] = cv[u];
            Rs[e] = sv[u];
        }
        __syncthreads();
        // per-head RMSNorm, then NeoX RoPE on (i, i + half) at position pos0 + b: one wave per row,
        // 4 dims per lane for the norm, then pair i per lane for the rotation (the wave's own LDS
        // writes are in order before its reads, so no barrier between the two)
        {
            const int nrow = QH + (has_new ? p.B : 0);
            for (int r = wv; r < nrow; r += ATT_NWV) {
                float *x = r < QH ? Qs[r] : Kn[r - QH];
                const float4 w = r < QH ? qw : kw;
                float4 v = *(const float4 *)(x + 4 * lane);
                const float sc = 1.0f / sqrtf(wave_sum64(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w) / (float)ATT_HD + p.eps);
                v = make_float4((v.x * sc) * w.x, (v.y * sc) * w.y, (v.z * sc) * w.z, (v.w * sc) * w.w);
                *(float4 *)(x + 4 * lane) = v;
                const int b = r < QH ? divp(r) : r - QH;
                for (int i = lane; i < p.half; i += 64) {
                    const float cs = Rc[b * p.half + i], sn = Rs[b * p.half + i];
                    const float v0 = x[i], v1 = x[i + p.half];
                    x[i] = v0 * cs - v1 * sn;
                    x[i + p.half] = v0 * sn + v1 * cs;
                }
            }
        }
        __syncthreads();
        // cache rows of the new positions this span holds (each position is in exactly one span)
        if (has_new && hh == 0)
            for (int e = tid; e < p.B * 64; e += ATT_NWV * 64) {
                const int b = e >> 6, d4 = e & 63, t = pos0 + b;
                if (t < posA || t >= posB) continue;
                const uint64_t row = (uint64_t)t * kvrow + hoff + 4 * d4;
                st_stream4(p.kc + row, *(const float4 *)&Kn[b][4 * d4]);
                st_stream4(p.vc + row, *(const float4 *)&Vn[b][4 * d4]);
            }
#pragma unroll
        for (int rt = 0; rt < NRT; rt++)
#pragma unroll
            for (int q = 0; q < ATT_NQ; q++) qop[rt][q] = *(const v4f *)&Qs[rt * 16 + n][d0 + 16 * q + 4 * gq];
        __syncthreads();                          // lds is the score exchange from here on
    }

    v4f oacc[NRT][ATT_NQ];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++)
#pragma unroll
        for (int c = 0; c < ATT_NQ; c++) oacc[rt][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // scores in log2 units: q.k / sqrt(hd) * log2(e), so probabilities are exp2 of differences
    const float scale = 1.4426950408889634f / sqrtf((float)ATT_HD);
    v4f *Sx = (v4f *)lds;                         // [2][ATT_NWV][NRT][64]
    const float *Sf = (const float *)lds;
    constexpr int SM_UPW = (NRT * 4 + ATT_NWV - 1) / ATT_NWV;    // softmax units per wave
    float sm[SM_UPW], sl[SM_UPW];
    int slim[SM_UPW];
#pragma unroll
    for (int j = 0; j < SM_UPW; j++) {
        const int R = 4 * (wv + j * ATT_NWV) + (lane >> 4);
        sm[j] = -INFINITY;
        sl[j] = 0.0f;
        slim[j] = R < QH ? pos0 + divp(R) : -1;
    }
    // K rows of new positions (FUSED: prepared in Kn, not in the caches yet) into slot kr_
    auto new_k = [&](int tt, v4f *kr_) {
        if (FUSED && tt * ATT_TP + ATT_TP - 1 >= pos0) {      // wave-uniform
            const int pp = tt * ATT_TP + n, b = min(max(pp - pos0, 0), p.B - 1);
#pragma unroll
            for (int q = 0; q < ATT_NQ; q++) {
                const v4f kn = *(const v4f *)&Kn[b][d0 + 16 * q + 4 * gq];
                if (pp >= pos0) kr_[q] = kn;
            }
        }
    };
    // partial score tiles of tile tt over this wave's dims, into exchange buffer bf
    // the K-index 8 gq + i of one 32-dim product stands for the dim d0 + 16 (i / 4) + 4 gq + i % 4 (pair
    // h of the wave's dims: h = q / 2), in the K operand (lane: position n) and the Q operand (lane: row
    // n) alike, so each product is a dot product over the wave's dims
    SplitH qsp[NRT][ATT_NQ / 2];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++)
#pragma unroll
        for (int h = 0; h < ATT_NQ / 2; h++) qsp[rt][h] = split_h8(qop[rt][2 * h], qop[rt][2 * h + 1]);
    auto scores = [&](const v4f *kr_, int bf) {
        SplitH ksp[ATT_NQ / 2];
#pragma unroll
        for (int h = 0; h < ATT_NQ / 2; h++) ksp[h] = split_h8(kr_[2 * h], kr_[2 * h + 1]);
#pragma unroll
        for (int rt = 0; rt < NRT; rt++) {
            v4f sp = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int h = 0; h < ATT_NQ / 2; h++) sp = mfma_split_h(ksp[h], qsp[rt][h], sp);
            Sx[((bf * ATT_NWV + wv) * NRT + rt) * SXS + lane + (lane >> 4)] = sp;
        }
    };
    new_k(tile0, kr[0]);
    scores(kr[0], 0);
    __syncthreads();
    // step t: loads of tile t + 2; the softmax of tile t (vector ALU), which reads the exchange
    // buffer the previous step filled, beside the scores of tile t + 1 (matrix cores) into the
    // other buffer; one barrier; then P.V of tile t.
    for (int t0 = tile0; t0 < tile1; t0 += NSL)
#pragma unroll
    for (int u = 0; u < NSL; u++) {
        const int t = t0 + u;
        if (t >= tile1) break;
        const int buf = (t - tile0) & 1;
        load_kv(t + 2, kr[(u + 2) % NSL], vr[(u + 2) % NSL], t + 2 < tile1);
        // softmax: unit su (rows 4 su .. 4 su + 3 of the block, 16 positions: one value per lane)
        // is owned by wave su % NWV, which keeps the running max / sum of its rows
#pragma unroll
        for (int j = 0; j < SM_UPW; j++) {
            const int su = wv + j * ATT_NWV;
            if (su < NRT * 4) {
                const int R = 4 * su + (lane >> 4), pq = lane & 15, rt = R >> 4, nr = R & 15;
                const int li = ((pq >> 2) * 17 + nr) * 4 + (pq & 3);     // float of lane (pq/4, nr), register pq%4 (padded)
                float sc = Sf[((buf * ATT_NWV + 0) * NRT + rt) * SXS * 4 + li];
#pragma unroll
                for (int w = 1; w < ATT_NWV; w++) sc += Sf[((buf * ATT_NWV + w) * NRT + rt) * SXS * 4 + li];
                const int pp = t * ATT_TP + pq;
                const float sv = pp <= slim[j] ? sc * scale : -INFINITY;
                const float mnew = fmaxf(sm[j], rowmax16(sv));
                const float alpha = mnew > -INFINITY ? __builtin_amdgcn_exp2f(sm[j] - mnew) : 1.0f;   // 0 for the first live tile
                const float pv = sv > -INFINITY ? __builtin_amdgcn_exp2f(sv - mnew) : 0.0f;
                sl[j] = sl[j] * alpha + rowsum16(pv);
                sm[j] = mnew;
                const int pi = (((buf * NRT + rt) * 4 + (pq >> 2)) * 16 + nr) * 4 + (pq & 3);
                const __bf16 ph = (__bf16)pv;
                Ph[pi] = __builtin_bit_cast(uint16_t, ph);
                Plo[pi] = __builtin_bit_cast(uint16_t, (__bf16)(pv - (float)ph));
                if (pq == 0) Al[buf * NRT * 16 + R] = alpha;
            }
        }
        if (t + 1 < tile1) {
            new_k(t + 1, kr[(u + 1) % NSL]);
            scores(kr[(u + 1) % NSL], buf ^ 1);
        }
        __syncthreads();
        if (FUSED && t * ATT_TP + ATT_TP - 1 >= pos0) {      // V rows of new positions, prepared in Vn
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int pv_ = t * ATT_TP + 4 * gq + v, bv = min(max(pv_ - pos0, 0), p.B - 1);
                const vqf vn = *(const vqf *)&Vn[bv][d0 + ATT_NQ * n];
                if (pv_ >= pos0) vr[u][v] = vn;
            }
        }
        // one 16-position product per output tile c, the K-index 4 gq + j standing for position 4 gq + j:
        // the lane's P operand is its four probabilities, its V operand the four v rows it loaded
        SplitB vsp[ATT_NQ];
#pragma unroll
        for (int c = 0; c < ATT_NQ; c++) vsp[c] = split_b4(vr[u][0][c], vr[u][1][c], vr[u][2][c], vr[u][3][c]);
#pragma unroll
        for (int rt = 0; rt < NRT; rt++) {
            const int pi = (((buf * NRT + rt) * 4 + gq) * 16 + n) * 4;
            const v4f al = *(const v4f *)&Al[buf * NRT * 16 + rt * 16 + 4 * gq];
            // rescale the O rows 4gq + w by their rows' factor
#pragma unroll
            for (int w = 0; w < 4; w++)
#pragma unroll
                for (int c = 0; c < ATT_NQ; c++) oacc[rt][c][w] *= al[w];
            const SplitB psp = { *(const v4s *)&Ph[pi], *(const v4s *)&Plo[pi] };
#pragma unroll
            for (int c = 0; c < ATT_NQ; c++) oacc[rt][c] = mfma_split_b(psp, vsp[c], oacc[rt][c]);
        }
    }
    // ---- partials of this span
    float *ml = p.pml + ((uint64_t)g * p.nspan + s) * ATT_MAXQ * 2;
    float *o = p.po + ((uint64_t)g * p.nspan + s) * ATT_MAXQ * ATT_HD;
#pragma unroll
    for (int j = 0; j < SM_UPW; j++) {
        const int R = 4 * (wv + j * ATT_NWV) + (lane >> 4);
        if ((lane & 15) == 0 && wv + j * ATT_NWV < NRT * 4 && R < QH) {
            const int rf = rfull(R);
            ml[2 * rf] = sm[j];
            ml[2 * rf + 1] = sl[j];
        }
    }
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const int r = rt * 16 + 4 * gq + w;
            if (r < QH) {
                vqf ov;
#pragma unroll
                for (int c = 0; c < ATT_NQ; c++) ov[c] = oacc[rt][c][w];
                *(vqf *)(o + (uint64_t)rfull(r) * ATT_HD + d0 + ATT_NQ * n) = ov;
            }
        }
    }
}

// out[b][h*hd + d] = sum_c o_c exp(m_c - M) / sum_c l_c exp(m_c - M) * sigmoid(gate) over the
// nc <= ATT_NSPAN spans with work (rows with no position in a span have m = -inf there and
// are skipped).  One wave per call: lane c holds the (m, l) of spans c, c + 64, ...; the max
// and the weighted sum of l are wave reductions, and the o loads are independent of them
// and of each other.
#define ATT_SPL ((ATT_NSPAN + 63) / 64)   // spans per lane in the combine
static __device__ __forceinline__ float combine_one(const float *q, uint64_t ldq, const float *pml, const float *po,
                                                    int nspan, int nc, int per, int h, int b, int d)
{
    const int lane = threadIdx.x & 63;
    const int g = h / per, qi = b * per + (h % per);
    const float *mlg = pml + (uint64_t)g * nspan * ATT_MAXQ * 2 + 2 * qi;
    const float *pog = po + (uint64_t)g * nspan * ATT_MAXQ * ATT_HD + (uint64_t)qi * ATT_HD + d;
    const float gate = q[(uint64_t)b * ldq + (uint64_t)h * 2 * ATT_HD + ATT_HD + d];
    // every o load of the call first, 16 spans at a step: they do not depend on the (m, l)
    // reduction, so the call waits for one memory latency.  Past nc a load repeats span nc - 1
    // (finite) and that span's weight f is 0 below, so the padding terms add 0.
    float ov[ATT_NSPAN];
#pragma unroll
    for (int c0 = 0; c0 < ATT_NSPAN; c0 += 16)
        if (c0 < nc)
#pragma unroll
            for (int j = 0; j < 16; j++)
                ov[c0 + j] = pog[(uint64_t)(c0 + j < nc ? c0 + j : nc - 1) * ATT_MAXQ * ATT_HD];
    float mc[ATT_SPL], lc[ATT_SPL], f[ATT_SPL];
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < ATT_SPL; u++) {
        const int c = lane + 64 * u;
        mc[u] = -INFINITY;
        lc[u] = 0.0f;
        if (c < nc) {
            mc[u] = mlg[(uint64_t)c * ATT_MAXQ * 2];
            lc[u] = mlg[(uint64_t)c * ATT_MAXQ * 2 + 1];
        }
        m = fmaxf(m, mc[u]);
    }
    m = wave_max64(m);
    float l = 0.0f;
#pragma unroll
    for (int u = 0; u < ATT_SPL; u++) {
        f[u] = mc[u] > -INFINITY ? __builtin_amdgcn_exp2f(mc[u] - m) : 0.0f;      // maxima in log2 units
        l += lc[u] * f[u];
    }
    l = wave_sum64(l);
    // sum over spans in order, 16 at a step (the o loads were all issued above)
    float acc = 0.0f;
#pragma unroll
    for (int c0 = 0; c0 < ATT_NSPAN; c0 += 16)
        if (c0 < nc) {
            const float fu = f[c0 >> 6];          // spans c0 .. c0 + 15 sit in f[c0 / 64]
#pragma unroll
            for (int j = 0; j < 16; j++)
                acc = fmaf(ov[c0 + j],
                           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, fu), (c0 + j) & 63)),
                           acc);
        }
    return (acc / l) * (1.0f / (1.0f + expf(-gate)));
}

// block (h, b): head h of token b, thread = dim
__global__ __launch_bounds__(ATT_HD) void k_attn_combine(const float *q, uint64_t ldq, const float *pml,
                                                         const float *po, const int *pos_dev, int B, int n_head,
                                                         int n_kv, int nspan, float *out, uint64_t ldo)
{
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    int ntl, tps, nc;
    span_split(*pos_dev, B, nspan, ntl, tps, nc);
    out[(uint64_t)b * ldo + (uint64_t)h * ATT_HD + d] = combine_one(q, ldq, pml, po, nspan, nc, n_head / n_kv, h, b, d);
}

// The combine with the output rows also written as the GEMV input digit planes
// (what the COPY preparation writes from them): block (h, b), thread = dim, merges
// head h of token b, whose 256 outputs are super-block h of the row; the block's
// maximum (one barrier) gives the token's shift, and tok_digits writes its digits.
// One token per block spreads the span partials' reads over n_head x B compute units.
__global__ __launch_bounds__(ATT_HD) void k_attn_combine_act(const float *q, uint64_t ldq, const float *pml,
                                                             const float *po, const int *pos_dev, int B,
                                                             int n_head, int n_kv, int nspan, float *out,
                                                             uint64_t ldo, uint8_t *A, float *xs)
{
    __shared__ float mxw[ATT_HD / 64];
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x, lane = d & 63;
    int ntl, tps, nc;
    span_split(*pos_dev, B, nspan, ntl, tps, nc);
    const float val = combine_one(q, ldq, pml, po, nspan, nc, n_head / n_kv, h, b, d);
    if (out) out[(uint64_t)b * ldo + (uint64_t)h * ATT_HD + d] = val;   // fp32 rows when asked for
    const float mw = wave_max64(fabsf(val));
    if (lane == 0) mxw[d >> 6] = mw;
    __syncthreads();
    const float mx = fmaxf(fmaxf(mxw[0], mxw[1]), fmaxf(mxw[2], mxw[3]));
    const int a = b >> 2;
    tok_digits(val, mx, b & 3, A + (uint64_t)a * PLANE_BYTES + (uint64_t)h * DIGIT_TILE,
               xs + (uint64_t)a * XS_FLOATS + (uint64_t)h * 16);
}

// The span-partial workspace is sized for the largest span count (ATT_NSPAN), so
// one reservation serves every later context length of that head count.  A
// larger head count (another model) takes a new buffer; the old one is kept,
// not freed, because HIP graphs captured earlier hold its address.
static bool attn_cache_fits(int ctx_bound, int n_kv)
{
    return (uint64_t)ctx_bound * (uint64_t)n_kv * ATT_HD * sizeof(float) <= ATT_RECORDS;
}
extern "C" int qgpu_attn_cache_fits(int ctx_bound, int n_kv)
{
    return ctx_bound >= 1 && n_kv >= 1 && attn_cache_fits(ctx_bound, n_kv);
}

static void *ws_attn_retired[16];
static int n_ws_attn_retired = 0;

static int attn_ws(int ctx_bound, int n_kv, int *nspan)
{
    // the K/V rows are read through buffer resources at 32-bit offsets from a kv head's row 0,
    // which reach ctx_bound * n_kv * ATT_HD floats: a cache beyond the resource is rejected
    if (!attn_cache_fits(ctx_bound, n_kv)) return QGPU_E_RANGE;
    const int nt = (ctx_bound + ATT_TP - 1) / ATT_TP;
    *nspan = nt < ATT_NSPAN ? nt : ATT_NSPAN;
    const size_t need = (size_t)n_kv * ATT_NSPAN * ATT_MAXQ * (2 + ATT_HD) * sizeof(float);
    if (need > qg::ws_attn_bytes) {
        void *p = nullptr;
        QG_CHECK(hipMalloc(&p, need));
        if (qg::ws_attn) {
            if (n_ws_attn_retired < 16) ws_attn_retired[n_ws_attn_retired++] = qg::ws_attn;
            // (beyond 16 retired buffers the oldest addresses are simply kept allocated)
        }
        qg::ws_attn = p;
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

// The head split: two span blocks per (kv head, span), each serving half of the kv head's query
// heads, where that takes fewer row tiles (6 heads x 3..8 tokens: 2 -> 1 or 3 -> 2) and the live
// context has few spans: 2 n_kv nsl <= compute units for every live context up to the bound
// returned, in positions (0: never).  Measured at 800 positions, 6 heads per kv head: B = 4 12.7 ->
// 11.2 us per call (span kernel + combine), B = 8 15.9 -> 14.1 us; at 8392 positions (236 span
// blocks already) it is 4% slower, and at B = 1 (one row tile either way) 20% slower.
#ifndef ATT_HSPLIT
#define ATT_HSPLIT 1
#endif
static int att_split_bound(int nspan, int B, int n_head, int n_kv)
{
    const int per = n_head / n_kv;
    if (!ATT_HSPLIT || per % 2 || (per * B + 15) / 16 <= ((per / 2) * B + 15) / 16 || qg::n_cu <= 0) return 0;
    if (2 * n_kv * nspan <= qg::n_cu) return INT_MAX;  // every span count qualifies
    int bound = 0;
    for (int pos = 0;; pos += ATT_TP) {               // live contexts pos + B, one tile at a time
        int ntl, tps, nsl;
        span_split(pos, B, nspan, ntl, tps, nsl);
        if (2 * n_kv * nsl > qg::n_cu) return bound;
        bound = ntl * ATT_TP;
    }
}

static int attn_launch(const AttnArgs &a0, int fused, int ctx_bound, float *out, uint64_t ldo, int act = 0,
                       int live_hi = 0)
{
    AttnArgs a = a0;
    int rc = attn_ws(ctx_bound, a.n_kv, &a.nspan);
    if (rc) return rc;
    a.pml = (float *)qg::ws_attn;
    a.po = a.pml + (size_t)a.n_kv * a.nspan * ATT_MAXQ * 2;
    const int hs = fused && live_hi >= a.B && live_hi <= att_split_bound(a.nspan, a.B, a.n_head, a.n_kv) ? 2 : 1;
    const int nrt = ((a.n_head / a.n_kv / hs) * a.B + 15) / 16;
    // 8 waves of 32 dims for one or two row tiles, 4 waves of 64 dims for three (same-box A/B: each
    // the faster one by ~0.5%)
    const int units = a.n_kv * a.nspan;
    const dim3 grid = hs == 1 ? dim3(a.n_kv, a.nspan) : dim3(16 * ((units + 7) / 8));
#define ATT_GO(F_, R_, H_) hipLaunchKernelGGL((k_attn_span<F_, R_, (R_ < 3 ? 8 : ATT_NW3), H_>), grid, \
                                              dim3((R_ < 3 ? 8 : ATT_NW3) * 64), 0, qg::stream, a)
#define ATT_RTS(F_) do { switch (nrt) { case 1: ATT_GO(F_, 1, 1); break; case 2: ATT_GO(F_, 2, 1); break; \
                         default: ATT_GO(F_, 3, 1); break; } } while (0)
    if (hs == 2) { if (nrt == 1) ATT_GO(1, 1, 2); else ATT_GO(1, 2, 2); }
    else if (fused) ATT_RTS(1);
    else ATT_RTS(0);
#undef ATT_RTS
#undef ATT_GO
    QG_LAUNCH_CHECK();
    if (act)
        hipLaunchKernelGGL(k_attn_combine_act, dim3(a.n_head, a.B), dim3(ATT_HD), 0, qg::stream, a.q,
                           a.ldq, a.pml, a.po, a.pos_dev, a.B, a.n_head, a.n_kv, a.nspan, out, ldo, (uint8_t *)qg::ws,
                           (float *)((uint8_t *)qg::ws + 2 * PLANE_BYTES));
    else
        hipLaunchKernelGGL(k_attn_combine, dim3(a.n_head, a.B), dim3(ATT_HD), 0, qg::stream, a.q, a.ldq, a.pml,
                           a.po, a.pos_dev, a.B, a.n_head, a.n_kv, a.nspan, out, ldo);
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

static int attn_fused(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                      const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                      const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev, int ctx_bound,
                      int B, int n_head, int n_kv, int head_dim, float eps, float *out, uint64_t ldo, int act,
                      int live_hi = 0)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (head_dim != ATT_HD) return QGPU_E_RANGE;
    if (!q || !k || !v || !q_norm_w || !k_norm_w || !kcache || !vcache || !rope_cos || !rope_sin || !pos_dev ||
        (!out && !act) || B < 1 || n_kv < 1 || n_head % n_kv || rope_dim < 2 || rope_dim > ATT_HD || rope_dim % 2 ||
        ctx_bound < B || ldq % 4 || ldkv % 4 || ((uintptr_t)q & 15) || ((uintptr_t)k & 15) || ((uintptr_t)v & 15) ||
        ((uintptr_t)kcache & 15) || ((uintptr_t)vcache & 15) || ((uintptr_t)q_norm_w & 15) ||
        ((uintptr_t)k_norm_w & 15))
        return QGPU_E_ARG;
    if ((n_head / n_kv) * B > ATT_MAXR || B > ATT_MAXB || (act && (uint64_t)n_head * ATT_HD > MAX_K))
        return QGPU_E_RANGE;
    AttnArgs a = {};
    a.q = q; a.ldq = ldq; a.k = k; a.v = v; a.ldkv = ldkv; a.qw = q_norm_w; a.kw = k_norm_w;
    a.rcos = rope_cos; a.rsin = rope_sin; a.kc = kcache; a.vc = vcache; a.pos_dev = pos_dev;
    a.half = rope_dim / 2; a.B = B; a.n_head = n_head; a.n_kv = n_kv; a.eps = eps;
    if (live_hi && (live_hi < B || live_hi > ctx_bound)) return QGPU_E_ARG;
    return attn_launch(a, 1, ctx_bound, out, ldo, act, live_hi);
}

extern "C" int qgpu_attn_fused(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                               const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                               const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev,
                               int ctx_bound, int B, int n_head, int n_kv, int head_dim, float eps, float *out,
                               uint64_t ldo)
{
    return attn_fused(q, ldq, k, v, ldkv, q_norm_w, k_norm_w, kcache, vcache, rope_cos, rope_sin, rope_dim, pos_dev,
                      ctx_bound, B, n_head, n_kv, head_dim, eps, out, ldo, 0);
}

extern "C" int qgpu_attn_fused_act(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                                   const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                                   const float *rope_cos, const float *rope_sin, int rope_dim, const int *pos_dev,
                                   int ctx_bound, int B, int n_head, int n_kv, int head_dim, float eps, float *out,
                                   uint64_t ldo)
{
    return attn_fused(q, ldq, k, v, ldkv, q_norm_w, k_norm_w, kcache, vcache, rope_cos, rope_sin, rope_dim, pos_dev,
                      ctx_bound, B, n_head, n_kv, head_dim, eps, out, ldo, 1);
}

extern "C" int qgpu_attn_fused_act_live(const float *q, uint64_t ldq, const float *k, const float *v, uint64_t ldkv,
                                        const float *q_norm_w, const float *k_norm_w, float *kcache, float *vcache,
                                        const float *rope_cos, const float *rope_sin, int rope_dim,
                                        const int *pos_dev, int ctx_bound, int B, int n_head, int n_kv, int head_dim,
                                        float eps, float *out, uint64_t ldo, int live_hi)
{
    return attn_fused(q, ldq, k, v, ldkv, q_norm_w, k_norm_w, kcache, vcache, rope_cos, rope_sin, rope_dim, pos_dev,
                      ctx_bound, B, n_head, n_kv, head_dim, eps, out, ldo, 1, live_hi);
}

extern "C" int qgpu_attn_split_bound(int ctx_bound, int B, int n_head, int n_kv)
{
    if (qg::ensure_init()) return 0;
    if (ctx_bound < 1 || B < 1 || n_kv < 1 || n_head % n_kv) return 0;
    const int nt = (ctx_bound + ATT_TP - 1) / ATT_TP, nspan = nt < ATT_NSPAN ? nt : ATT_NSPAN;
    const int b = att_split_bound(nspan, B, n_head, n_kv);
    return b < ctx_bound ? b : ctx_bound;
}

// Reserve the attention workspace up front (so later calls never allocate,
// e.g. inside a captured graph): ctx_bound positions, n_kv heads.
extern "C" int qgpu_attn_reserve(int ctx_bound, int n_kv)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (ctx_bound < 1 || n_kv < 1) return QGPU_E_ARG;
    int nspan;
    return attn_ws(ctx_bound, n_kv, &nspan);
}
