// Batched dequant-GEMV for the ggml formats of the model (gfx950).
//
// IQ4_XS (the bulk of the weights) runs on the matrix cores:
//   * weights are repacked once into 16-row tiles; per (tile, 256-element
//     super-block) a 2176-byte record holds the 16 row headers (d, scales_h,
//     scales_l: 8 B each) and the 2048 nibble bytes arranged so that lane l of
//     a wave loads its MFMA B operand for 4 sub-blocks with one 16-byte load;
//   * a nibble dword decodes with 4 v_perm_b32 into two int8 halves of the
//     codebook values, which two chained MFMAs multiply by the same operand;
//   * the activations are turned once per call into 3 balanced int8 "digits"
//     of a 22-bit fixed-point value per (token, super-block):
//       x = 2^-s * (d0 + 2^8 d1 + 2^16 d2),  |x| 2^s < 2^22,
//     so v_mfma_i32_16x16x32_i8 computes exact integer sub-block dot products
//     for 4 tokens x 4 digit rows (rows of the A tile; the fourth digit row is
//     zero and is not stored or loaded) against 16 weight rows;
//   * the 6-bit sub-block scale (ls - 32) is applied in int32 (exact: |acc| <
//     2^27 per super-block), then (d * 2^(8 dgt - s)) once per super-block in
//     fp32.  The roundings are the x quantisation (2^-23 of the super-block
//     max) and the fp32 super-block accumulation.
// Q4_K/Q5_K/Q6_K/Q8_0 run on the same matrix-core path; F32 (and Q8_0 rows
// that are not a multiple of 256) use a VALU kernel on the GGUF layout.
#include "qgpu_internal.h"
#include <stdlib.h>

typedef int v4i __attribute__((ext_vector_type(4)));

#define RSS_FLOATS  ((size_t)QGPU_MAX_B * MAX_NSB)
#define ACT_RMS_DEFER 4      // internal prep kind: RMSNORM with the 1/rms factor applied by the GEMV
#define ACT_RMS_EMBD 5       // ACT_RMS_DEFER on rows gathered from the embedding matrix
#define ACT_RMS_CAT 6        // the two-segment RMSNORM [x | y] with both row factors applied by the GEMV

// Pair split (tail balance): when a launch's tiles are a little over a multiple of the compute
// units, the remainder tiles run as two half-K blocks each, whose results meet in 64-bit exchange
// slots (PAIR_SLOTS per tile).  The slots hold 0 between launches.
#define PAIR_MAX_TILES 256
#define PAIR_SLOTS     (QGPU_MAX_B / 4 * 64)          // (plane, token, row) entries of one tile
#define XCHG_BYTES     ((size_t)PAIR_MAX_TILES * PAIR_SLOTS * sizeof(unsigned long long))
#define GEMV_WS_XCHG   (2 * PLANE_BYTES + 2 * XS_FLOATS * sizeof(float) + RSS_FLOATS * sizeof(float))
#define GEMV_WS_BYTES  (GEMV_WS_XCHG + XCHG_BYTES)
size_t qg_gemv_workspace_bytes() { return GEMV_WS_BYTES; }

// Where a GEMV runs: its stream and its activation workspace (two digit planes,
// their conversion factors, the deferred-RMSNorm sums).  The library entry
// points use the library stream and workspace; qgpu_gemv_batch_noalloc the
// caller's stream and a static device array.
struct GemvExec {
    hipStream_t st;
    uint8_t *ws;
    int n_cu;            // compute units of the device (0: no pair split)
};
static GemvExec lib_exec() { return GemvExec{ qg::stream, (uint8_t *)qg::ws, qg::n_cu }; }
static unsigned long long *ws_xchg(const GemvExec &ex) { return (unsigned long long *)(ex.ws + GEMV_WS_XCHG); }
static float *ws_rss(const GemvExec &ex) { return (float *)(ex.ws + 2 * PLANE_BYTES + 2 * XS_FLOATS * sizeof(float)); }

static __device__ __forceinline__ float h2f(uint32_t h16) { return (float)__builtin_bit_cast(_Float16, (unsigned short)h16); }

// ---------------------------------------------------------------- repack
// Row header re-arrangement (lossless, same 8 bytes).  GGUF: d | scales_h | scales_l[4]
// with ls_ib = nibble ib of scales_l | 2 bits ib of scales_h << 4.  Packed: the
// six-bit two's-complement value s_ib = ls_ib ^ 32 (= ls_ib - 32 mod 64) of
// every sub-block at a fixed bit offset, so one signed bit-field extract yields
// (ls - 32):
//   x = d | s5 << 16 | s6 << 22 | (s7 & 15) << 28
//   y = s0 | s1 << 6 | s2 << 12 | s3 << 18 | s4 << 24 | (s7 >> 4) << 30
static __device__ __forceinline__ uint2 hdr_pack(uint2 raw)
{
    const uint32_t sh = raw.x >> 16, sl = raw.y;
    uint32_t sv[8];
#pragma unroll
    for (int ib = 0; ib < 8; ib++) sv[ib] = ((((sl >> (4 * ib)) & 15u) | (((sh >> (2 * ib)) & 3u) << 4)) ^ 32u);
    uint2 o;
    o.x = (raw.x & 0xFFFFu) | (sv[5] << 16) | (sv[6] << 22) | ((sv[7] & 15u) << 28);
    o.y = sv[0] | (sv[1] << 6) | (sv[2] << 12) | (sv[3] << 18) | (sv[4] << 24) | ((sv[7] >> 4) << 30);
    return o;
}
static __device__ __forceinline__ uint32_t hdr_s6(uint2 h, int ib)   // unsigned 6-bit s_ib
{
    if (ib < 5) return (h.y >> (6 * ib)) & 63u;
    if (ib < 7) return (h.x >> (16 + 6 * (ib - 5))) & 63u;
    return (h.x >> 28) | ((h.y >> 30) << 4);
}
static __device__ __forceinline__ int hdr_scale(uint2 h, int ib)     // ls_ib - 32
{
    return ((int)(hdr_s6(h, ib) << 26)) >> 26;
}
static __device__ __forceinline__ uint2 hdr_unpack(uint2 h)
{
    uint32_t sh = 0, sl = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
        const uint32_t ls = hdr_s6(h, ib) ^ 32u;
        sl |= (ls & 15u) << (4 * ib);
        sh |= (ls >> 4) << (2 * ib);
    }
    return make_uint2((h.x & 0xFFFFu) | (sh << 16), sl);
}

// raw (GGUF rows of nsb 136-byte super-blocks) <-> tile records.
// packed dword (row n, lane group g, sub-block ib) of record (T, s) at
//   128 + ((ib/4)*64 + g*16 + n)*16 + (ib%4)*4  and holds qs bytes 4g..4g+3 of sub-block ib.
__global__ void k_repack_iq4(const uint8_t *__restrict__ raw, uint8_t *__restrict__ pk, uint64_t ne1,
                             uint32_t nsb, uint64_t rows_pad, int unpack)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows_pad * nsb) return;
    const uint64_t r = i / nsb;
    const uint32_t s = (uint32_t)(i % nsb);
    const uint64_t T = r / IQ4_TILE_ROWS;
    const uint32_t n = (uint32_t)(r % IQ4_TILE_ROWS);
    uint8_t *rec = pk + (T * nsb + s) * IQ4_REC_BYTES;
    const uint64_t rb = (uint64_t)nsb * 136;
    if (unpack) {
        if (r >= ne1) return;
        uint8_t *blk = (uint8_t *)raw + r * rb + (uint64_t)s * 136;
        *(uint2 *)blk = hdr_unpack(*(const uint2 *)(rec + n * 8));
        for (int ib = 0; ib < 8; ib++)
            for (int g = 0; g < 4; g++)
                *(uint32_t *)(blk + 8 + 16 * ib + 4 * g) =
                    *(const uint32_t *)(rec + IQ4_HDR_BYTES + ((ib / 4) * 64 + g * 16 + n) * 16 + (ib % 4) * 4);
        return;
    }
    const uint8_t *blk = raw + r * rb + (uint64_t)s * 136;
    const bool live = r < ne1;
    *(uint2 *)(rec + n * 8) = live ? hdr_pack(*(const uint2 *)blk) : make_uint2(0, 0);
    for (int ib = 0; ib < 8; ib++)
        for (int g = 0; g < 4; g++)
            *(uint32_t *)(rec + IQ4_HDR_BYTES + ((ib / 4) * 64 + g * 16 + n) * 16 + (ib % 4) * 4) =
                live ? *(const uint32_t *)(blk + 8 + 16 * ib + 4 * g) : 0u;
}

int qg_repack_iq4xs(const void *raw, uint64_t ne0, uint64_t ne1, void *packed, int unpack)
{
    const uint32_t nsb = (uint32_t)(ne0 / 256);
    const uint64_t rows_pad = (ne1 + IQ4_TILE_ROWS - 1) / IQ4_TILE_ROWS * IQ4_TILE_ROWS;
    const uint64_t n = rows_pad * nsb;
    hipLaunchKernelGGL(k_repack_iq4, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, qg::stream,
                       (const uint8_t *)raw, (uint8_t *)packed, ne1, nsb, rows_pad, unpack);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

// ---------------------------------------------------------------- K-quant and Q8_0 records
// Every packed format keeps the IQ4_XS nibble arrangement for its low four
// bits: per sub-block ib (32 elements), "virtual byte" j < 16 holds element j
// in its low nibble and element j + 16 in its high nibble, and dword
// (row n, lane group g, ib) at KQ_Q + ((ib/4)*64 + g*16 + n)*16 + (ib%4)*4
// holds virtual bytes 4g..4g+3.  Lane l = 16 g + n then loads its MFMA B
// operand of four sub-blocks with one 16-byte load, K-slot 8g+c standing for
// element 4g+c and slot 8g+4+c for element 16+4g+c, exactly as the activation
// digits are laid out.  Per format:
//   Q4_K  [0,256)     row n: d | dmin << 16, scales and mins as 6-bit fields
//                     (sc0..sc4 | m7 bits 0-1 << 30), (m0..m4 | m7 bits 2-3 << 30),
//                     (sc5, sc6, sc7, m5, m6 | m7 bits 4-5 << 30)
//         [256,2304)  nibbles
//   Q5_K  as Q4_K, then [2304,2816): lane l's 8 bytes at 2304 + 8 l, byte ib =
//                     fifth bits of its elements 4g+c (bits 0-3) and 16+4g+c (bits 4-7)
//   Q6_K  [0,256)     row n: the 16 int8 scales; [256,288) row n: fp16 d at 256 + 2n
//         [288,2336)  low nibbles
//         [2336,3360) lane l's 16 bytes at 2336 + 16 l: dword ib/2, byte c, bit pair
//                     4 (ib%2) + {0: element 4g+c, 2: element 16+4g+c} = top two bits
//   Q8_0  [0,256)     row n: the 8 fp16 d of its 32-element blocks
//         [256,4352)  lane l's 64 bytes at 256 + (p*64 + l)*16, p < 4: int8 elements
//                     4g..4g+3, 16+4g..16+4g+3 of sub-block 2p, then of sub-block 2p+1
#define KQ_HB5 2304
#define KQ_D6  256
#define KQ_Q6  288
#define KQ_HB6 2336
#define KQ_Q   256

static __device__ __forceinline__ uint32_t kq_qoff(int fmt, int n, int g, int ib)
{
    return (fmt == T_Q6_K ? KQ_Q6 : KQ_Q) + ((ib / 4) * 64 + g * 16 + n) * 16 + (ib % 4) * 4;
}

// get_scale_min_k4 of the reference (quant.h:21-29) for all eight sub-blocks
static __device__ __forceinline__ void kq_scales(const uint8_t *sc12, uint32_t sc[8], uint32_t m[8])
{
    for (int j = 0; j < 8; j++) {
        if (j < 4) { sc[j] = sc12[j] & 63; m[j] = sc12[j + 4] & 63; }
        else {
            sc[j] = (sc12[j + 4] & 15) | ((sc12[j - 4] >> 6) << 4);
            m[j] = (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4);
        }
    }
}
static __device__ __forceinline__ uint4 kq_hdr_pack(uint32_t dd, const uint32_t sc[8], const uint32_t m[8])
{
    uint4 h;
    h.x = dd;
    h.y = sc[0] | (sc[1] << 6) | (sc[2] << 12) | (sc[3] << 18) | (sc[4] << 24) | ((m[7] & 3u) << 30);
    h.z = m[0] | (m[1] << 6) | (m[2] << 12) | (m[3] << 18) | (m[4] << 24) | (((m[7] >> 2) & 3u) << 30);
    h.w = sc[5] | (sc[6] << 6) | (sc[7] << 12) | (m[5] << 18) | (m[6] << 24) | ((m[7] >> 4) << 30);
    return h;
}
static __device__ __forceinline__ uint32_t kq_sc(uint4 h, int ib)
{
    return ib < 5 ? (h.y >> (6 * ib)) & 63u : (h.w >> (6 * (ib - 5))) & 63u;
}
static __device__ __forceinline__ uint32_t kq_m(uint4 h, int ib)
{
    if (ib < 5) return (h.z >> (6 * ib)) & 63u;
    if (ib < 7) return (h.w >> (18 + 6 * (ib - 5))) & 63u;
    return (h.y >> 30) | ((h.z >> 30) << 2) | ((h.w >> 30) << 4);
}

// One thread per (row, super-block): GGUF block(s) <-> this row's slices of the record.
template <int FMT>
__global__ void k_repack_kq(const uint8_t *__restrict__ raw, uint8_t *__restrict__ pk, uint64_t ne1, uint32_t nsb,
                            uint64_t rows_pad, int unpack)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows_pad * nsb) return;
    const uint64_t r = i / nsb;
    const uint32_t s = (uint32_t)(i % nsb);
    const uint32_t n = (uint32_t)(r % IQ4_TILE_ROWS);
    const uint32_t BS = FMT == T_Q4_K ? 144 : FMT == T_Q5_K ? 176 : FMT == T_Q6_K ? 210 : 8 * 34;
    uint8_t *rec = pk + ((r / IQ4_TILE_ROWS) * nsb + s) * packed_rec_bytes(FMT);
    if (unpack && r >= ne1) return;
    const bool live = r < ne1;
    uint8_t *blk = (uint8_t *)raw + (live ? r * nsb * (uint64_t)BS + (uint64_t)s * BS : 0);
    // element values of the super-block: low four bits lo4[e], upper bits hi[e] (Q5_K 1, Q6_K 2), Q8_0 bytes
    uint8_t lo4[256], hi[256];
    if (!unpack) {
        if (FMT == T_Q8_0) {
            for (int b = 0; b < 8; b++)
                for (int e = 0; e < 32; e++) lo4[32 * b + e] = live ? blk[34 * b + 2 + e] : 0;
        } else if (FMT == T_Q6_K) {
            for (int e = 0; e < 256; e++) {
                const int h = e / 128, qt = (e % 128) / 32, l = e % 32;
                const uint8_t qlb = live ? blk[64 * h + (qt & 1) * 32 + l] : 0, qhb = live ? blk[128 + 32 * h + l] : 0;
                lo4[e] = (qt < 2) ? (qlb & 15) : (qlb >> 4);
                hi[e] = (qhb >> (2 * qt)) & 3;
            }
        } else {
            const uint8_t *qs = blk + (FMT == T_Q5_K ? 48 : 16);
            for (int e = 0; e < 256; e++) {
                const int ib = e / 32, ep = e % 32;
                const uint8_t b = live ? qs[32 * (ib / 2) + ep] : 0;
                lo4[e] = (ib & 1) ? (b >> 4) : (b & 15);
                hi[e] = FMT == T_Q5_K && live ? (blk[16 + ep] >> ib) & 1 : 0;
            }
        }
        // headers
        if (FMT == T_Q4_K || FMT == T_Q5_K) {
            uint32_t sc[8], m[8];
            kq_scales(blk + 4, sc, m);
            *(uint4 *)(rec + n * 16) = live ? kq_hdr_pack(*(const uint32_t *)blk, sc, m) : make_uint4(0, 0, 0, 0);
        } else if (FMT == T_Q6_K) {
            for (int j = 0; j < 16; j++) rec[n * 16 + j] = live ? blk[192 + j] : 0;
            *(uint16_t *)(rec + KQ_D6 + 2 * n) = live ? *(const uint16_t *)(blk + 208) : 0;
        } else {
            for (int b = 0; b < 8; b++) *(uint16_t *)(rec + n * 16 + 2 * b) = live ? *(const uint16_t *)(blk + 34 * b) : 0;
        }
        // quants
        for (int ib = 0; ib < 8; ib++)
            for (int g = 0; g < 4; g++) {
                if (FMT == T_Q8_0) {
                    uint8_t *q = rec + KQ_Q + ((ib / 2) * 64 + g * 16 + n) * 16 + (ib & 1) * 8;
                    for (int c = 0; c < 4; c++) { q[c] = lo4[32 * ib + 4 * g + c]; q[4 + c] = lo4[32 * ib + 16 + 4 * g + c]; }
                    continue;
                }
                uint32_t w = 0;
                for (int c = 0; c < 4; c++)
                    w |= (uint32_t)(lo4[32 * ib + 4 * g + c] | (lo4[32 * ib + 16 + 4 * g + c] << 4)) << (8 * c);
                *(uint32_t *)(rec + kq_qoff(FMT, n, g, ib)) = w;
                if (FMT == T_Q5_K) {
                    uint32_t b = 0;
                    for (int c = 0; c < 4; c++) b |= (uint32_t)(hi[32 * ib + 4 * g + c] << c) | (uint32_t)(hi[32 * ib + 16 + 4 * g + c] << (4 + c));
                    rec[KQ_HB5 + (g * 16 + n) * 8 + ib] = (uint8_t)b;
                }
                if (FMT == T_Q6_K) {
                    uint8_t *hb = rec + KQ_HB6 + (g * 16 + n) * 16 + (ib / 2) * 4;
                    for (int c = 0; c < 4; c++) {
                        const uint32_t v = hi[32 * ib + 4 * g + c] | (hi[32 * ib + 16 + 4 * g + c] << 2);
                        hb[c] = (uint8_t)((hb[c] & ~(15u << (4 * (ib & 1)))) | (v << (4 * (ib & 1))));
                    }
                }
            }
        return;
    }
    // unpack: gather the element values back, then write the GGUF block(s)
    for (int ib = 0; ib < 8; ib++)
        for (int g = 0; g < 4; g++) {
            if (FMT == T_Q8_0) {
                const uint8_t *q = rec + KQ_Q + ((ib / 2) * 64 + g * 16 + n) * 16 + (ib & 1) * 8;
                for (int c = 0; c < 4; c++) { lo4[32 * ib + 4 * g + c] = q[c]; lo4[32 * ib + 16 + 4 * g + c] = q[4 + c]; }
                continue;
            }
            const uint32_t w = *(const uint32_t *)(rec + kq_qoff(FMT, n, g, ib));
            for (int c = 0; c < 4; c++) {
                lo4[32 * ib + 4 * g + c] = (w >> (8 * c)) & 15;
                lo4[32 * ib + 16 + 4 * g + c] = (w >> (8 * c + 4)) & 15;
            }
            if (FMT == T_Q5_K) {
                const uint32_t b = rec[KQ_HB5 + (g * 16 + n) * 8 + ib];
                for (int c = 0; c < 4; c++) { hi[32 * ib + 4 * g + c] = (b >> c) & 1; hi[32 * ib + 16 + 4 * g + c] = (b >> (4 + c)) & 1; }
            }
            if (FMT == T_Q6_K) {
                const uint8_t *hb = rec + KQ_HB6 + (g * 16 + n) * 16 + (ib / 2) * 4;
                for (int c = 0; c < 4; c++) {
                    const uint32_t v = hb[c] >> (4 * (ib & 1));
                    hi[32 * ib + 4 * g + c] = v & 3;
                    hi[32 * ib + 16 + 4 * g + c] = (v >> 2) & 3;
                }
            }
        }
    if (FMT == T_Q8_0) {
        for (int b = 0; b < 8; b++) {
            *(uint16_t *)(blk + 34 * b) = *(const uint16_t *)(rec + n * 16 + 2 * b);
            for (int e = 0; e < 32; e++) blk[34 * b + 2 + e] = lo4[32 * b + e];
        }
    } else if (FMT == T_Q6_K) {
        for (int j = 0; j < 16; j++) blk[192 + j] = rec[n * 16 + j];
        *(uint16_t *)(blk + 208) = *(const uint16_t *)(rec + KQ_D6 + 2 * n);
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                const int e0 = 128 * h + l;
                blk[64 * h + l] = (uint8_t)(lo4[e0] | (lo4[e0 + 64] << 4));
                blk[64 * h + 32 + l] = (uint8_t)(lo4[e0 + 32] | (lo4[e0 + 96] << 4));
                blk[128 + 32 * h + l] = (uint8_t)(hi[e0] | (hi[e0 + 32] << 2) | (hi[e0 + 64] << 4) | (hi[e0 + 96] << 6));
            }
    } else {
        const uint4 h = *(const uint4 *)(rec + n * 16);
        *(uint32_t *)blk = h.x;
        uint32_t sc[8], m[8];
        for (int j = 0; j < 8; j++) { sc[j] = kq_sc(h, j); m[j] = kq_m(h, j); }
        uint8_t *s12 = blk + 4;
        for (int j = 0; j < 4; j++) {
            s12[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            s12[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
            s12[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t *qs = blk + (FMT == T_Q5_K ? 48 : 16);
        for (int j = 0; j < 4; j++)
            for (int ep = 0; ep < 32; ep++) qs[32 * j + ep] = (uint8_t)(lo4[64 * j + ep] | (lo4[64 * j + 32 + ep] << 4));
        if (FMT == T_Q5_K)
            for (int ep = 0; ep < 32; ep++) {
                uint32_t b = 0;
                for (int ib = 0; ib < 8; ib++) b |= (uint32_t)hi[32 * ib + ep] << ib;
                blk[16 + ep] = (uint8_t)b;
            }
    }
}

// packed <-> GGUF rows for every packed format (unpack = 1: packed -> raw)
int qg_repack(int type, const void *raw, uint64_t ne0, uint64_t ne1, void *packed, int unpack)
{
    if (type == T_IQ4_XS) return qg_repack_iq4xs(raw, ne0, ne1, packed, unpack);
    const uint32_t nsb = (uint32_t)(ne0 / 256);
    const uint64_t rows_pad = (ne1 + IQ4_TILE_ROWS - 1) / IQ4_TILE_ROWS * IQ4_TILE_ROWS;
    const uint64_t n = rows_pad * nsb;
    const dim3 grid((unsigned)((n + 63) / 64)), blk(64);
    switch (type) {
    case T_Q4_K: hipLaunchKernelGGL(k_repack_kq<T_Q4_K>, grid, blk, 0, qg::stream, (const uint8_t *)raw, (uint8_t *)packed, ne1, nsb, rows_pad, unpack); break;
    case T_Q5_K: hipLaunchKernelGGL(k_repack_kq<T_Q5_K>, grid, blk, 0, qg::stream, (const uint8_t *)raw, (uint8_t *)packed, ne1, nsb, rows_pad, unpack); break;
    case T_Q6_K: hipLaunchKernelGGL(k_repack_kq<T_Q6_K>, grid, blk, 0, qg::stream, (const uint8_t *)raw, (uint8_t *)packed, ne1, nsb, rows_pad, unpack); break;
    case T_Q8_0: hipLaunchKernelGGL(k_repack_kq<T_Q8_0>, grid, blk, 0, qg::stream, (const uint8_t *)raw, (uint8_t *)packed, ne1, nsb, rows_pad, unpack); break;
    default: return QGPU_E_TYPE;
    }
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

// ---------------------------------------------------------------- activation prep
// Digit planes: plane a holds tokens 4a..4a+3; the A tile of super-block sb is
// at A + a*PLANE_BYTES + sb*DIGIT_TILE and its factors at xs + a*XS_FLOATS + sb*16
// (layout: act_digits in qgpu_internal.h).
struct ActDev {
    const float *x, *y, *w, *w2;
    float *xout;
    uint64_t ldx, ldy, ldxo, seg;
    float eps;
    int ntok, digits;
    // ACT_RMS_DEFER: x_eff = x + sum of n_part partial planes (part + q*pstride + t*ldp), written
    // back to xnew when set (may alias x: a block reads and writes only its own super-block);
    // rss[t*nsb + sb] = sum over the super-block of x_eff^2
    const float *part;
    uint64_t ldp, pstride, ldxn;
    int n_part, nsb;
    float *xnew, *rss;
    // x (the first segment of the two-segment RMSNORM) gathered from rows tok[t] of a packed
    // IQ4_XS matrix of embd_ne1 rows instead of read from x
    const uint8_t *embd;
    const uint32_t *tok;
    uint64_t embd_ne1;
};

// Elements k..k+3 (k % 4 == 0) of row r of a packed IQ4_XS matrix with ne0 columns, as
// k_dequant_rows computes them (zeros for r >= ne1): the four share one dword of
// nibbles and one sub-block scale.
static __device__ __forceinline__ float4 embd_iq4x4(const uint8_t *W, uint64_t ne0, uint64_t ne1, uint32_t r,
                                                    uint64_t k)
{
    if (r >= ne1) return make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const uint32_t nsb = (uint32_t)(ne0 / 256), sb = (uint32_t)(k >> 8), ib = (uint32_t)(k >> 5) & 7;
    const uint32_t j = (uint32_t)k & 31, n = r % IQ4_TILE_ROWS;
    const uint8_t *rec = W + ((uint64_t)(r / IQ4_TILE_ROWS) * nsb + sb) * IQ4_REC_BYTES;
    const uint2 hdr = *(const uint2 *)(rec + n * 8);
    const float dl = __fmul_rn(h2f(hdr.x & 0xFFFFu), (float)hdr_scale(hdr, (int)ib));
    const uint32_t nib = (*(const uint32_t *)(rec + IQ4_HDR_BYTES + ((ib / 4) * 64 + ((j & 15) >> 2) * 16 + n) * 16 +
                                              (ib % 4) * 4) >> (j >= 16 ? 4 : 0)) & 0x0F0F0F0Fu;
    // the codebook (-127 -104 -83 -65 | -49 -35 -22 -10 | 1 13 25 38 | 53 69 89 113) as int8 bytes:
    // one byte permute per half, the half picked by bit 3 of each nibble
    const uint32_t sel = nib & 0x07070707u, hm = ((nib >> 3) & 0x01010101u) * 0xFFu;
    const uint32_t lo = __builtin_amdgcn_perm(0xF6EADDCFu, 0xBFAD9881u, sel);
    const uint32_t hi = __builtin_amdgcn_perm(0x71594535u, 0x26190D01u, sel);
    const uint32_t b = (lo & ~hm) | (hi & hm);
    return make_float4(__fmul_rn(dl, (float)(int8_t)(b & 0xFFu)), __fmul_rn(dl, (float)(int8_t)((b >> 8) & 0xFFu)),
                       __fmul_rn(dl, (float)(int8_t)((b >> 16) & 0xFFu)), __fmul_rn(dl, (float)(int8_t)(b >> 24)));
}

static __device__ __forceinline__ float embd_iq4(const uint8_t *W, uint64_t ne0, uint64_t ne1, uint32_t r, uint64_t k)
{
    const float4 v = embd_iq4x4(W, ne0, ne1, r, k & ~(uint64_t)3);
    const uint32_t c = (uint32_t)k & 3;
    return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

static __device__ __forceinline__ float silu_dev(float v) { return v / (1.0f + expf(-v)); }


// Row RMSNorm over a whole row or over each of its two segments (the MTP input
// concat(enorm(e), hnorm(h))).  One block = one 256-element super-block
// (blockIdx.x) of the 4 tokens of plane blockIdx.y; each block recomputes the row
// RMS of its segment in the same order, so every block gets the same value.  The
// four tokens' loads are issued before their first use.
template <bool GATH>
__global__ __launch_bounds__(256) void k_prep_rms(ActDev p, uint8_t *__restrict__ A, float *__restrict__ xs)
{
    __shared__ ActDigitLds dl;
    __shared__ float red[4][4];          // sums of squares [token][wave]
    const int e = threadIdx.x, sb = blockIdx.x, a = blockIdx.y;
    const int lane = e & 63, wv = e >> 6;
    const uint64_t k = (uint64_t)sb * 256 + e;
    const int nt = p.ntok - 4 * a < 4 ? p.ntok - 4 * a : 4;      // tokens of this plane (>= 1)
    int tr[4];                                                     // row of token i (clamped: always loadable)
#pragma unroll
    for (int i = 0; i < 4; i++) tr[i] = 4 * a + (i < nt ? i : 0);
    float v[4], m[4];
    const uint64_t segl = p.seg;
    const int part = (uint64_t)sb * 256 >= segl ? 1 : 0;
    const float *src = part ? p.y : p.x;
    const float *w = part ? p.w2 : p.w;
    const uint64_t ld = part ? p.ldy : p.ldx, kk = k - (part ? segl : 0);
    const bool gath = GATH && !part;                                // x rows from the embedding matrix
    uint32_t er[4];
#pragma unroll
    for (int i = 0; i < 4; i++) er[i] = gath ? p.tok[tr[i]] : 0u;
    float own[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        own[i] = gath ? embd_iq4(p.embd, segl, p.embd_ne1, er[i], kk) : src[(uint64_t)tr[i] * ld + kk];
    const float wk = w[kk];
    float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint64_t j0 = e; j0 < segl / 4; j0 += 5 * 256) {
        float4 q[5][4];
#pragma unroll
        for (int u = 0; u < 5; u++) {
            const uint64_t j = j0 + (uint64_t)u * 256;
#pragma unroll
            for (int i = 0; i < 4; i++)
                q[u][i] = (i < nt && j < segl / 4)
                              ? (gath ? embd_iq4x4(p.embd, segl, p.embd_ne1, er[i], 4 * j)
                                      : ((const float4 *)(src + (uint64_t)(4 * a + i) * ld))[j])
                              : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 5; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ss[i] = fmaf(q[u][i].x, q[u][i].x, ss[i]); ss[i] = fmaf(q[u][i].y, q[u][i].y, ss[i]);
                ss[i] = fmaf(q[u][i].z, q[u][i].z, ss[i]); ss[i] = fmaf(q[u][i].w, q[u][i].w, ss[i]);
            }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) ss[i] = wave_sum64(ss[i]);
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < 4; i++) red[i][wv] = ss[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float tot = (red[i][0] + red[i][1]) + (red[i][2] + red[i][3]);
        const float sc = 1.0f / sqrtf(tot / (float)segl + p.eps);
        v[i] = i < nt ? (own[i] * sc) * wk : 0.0f;
    }
    if (p.xout) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (i < nt) p.xout[(uint64_t)(4 * a + i) * p.ldxo + k] = v[i];
    }
    if (!p.digits) return;               // fp32 rows only (VALU formats)
#pragma unroll
    for (int i = 0; i < 4; i++) m[i] = wave_max64(fabsf(v[i]));
    act_digits(v, m, dl, A + (uint64_t)a * PLANE_BYTES + (uint64_t)sb * DIGIT_TILE, xs + (uint64_t)a * XS_FLOATS + (uint64_t)sb * 16);
}

// One token per block: the deferred RMSNorm (with the residual's pending partial
// planes), SiLU(x)·y, the per-head gated norm, and the plain copy.  Block (sb, t),
// 256 threads: thread e holds element e of super-block sb of token t, so a thread
// issues 1 + NP + 1 loads (deferred RMSNorm with NP partial planes), 2 or 3 (the
// others), with no branch around them; tok_digits writes token t's digits of the
// super-block straight from registers.  One barrier exchanges the
// per-wave sums of squares and maxima (the gated norm takes two: its maximum
// follows the head scale).  The per-element arithmetic and the reduction orders
// are those of the 4-token form (wave sums, then (w0 + w1) + (w2 + w3)), so
// digits, scales, sums of squares and residual rows do not depend on the grid.
template <int KIND, int NP>
__global__ __launch_bounds__(256) void k_prep_tok(ActDev p, uint8_t *__restrict__ A, float *__restrict__ xs)
{
    __shared__ float ssw[4], mxw[4];
    const int e = threadIdx.x, lane = e & 63, wv = e >> 6;
    const int sb = blockIdx.x, t = blockIdx.y, a = t >> 2, i = t & 3;
    const uint32_t k = (uint32_t)sb * 256 + e;
    float v, ss = 0.0f;
    constexpr bool RMS = KIND == ACT_RMS_DEFER || KIND == ACT_RMS_EMBD || KIND == ACT_RMS_CAT;
    if (KIND == ACT_RMS_CAT) {
        // [x | y], seg elements each: v = x * w or y * w2 (its segment's row factor is the GEMV's),
        // and the super-block's sum of squares of x or y; x from the embedding rows when embd is set
        const uint32_t segl = (uint32_t)p.seg;
        const bool s1 = k >= segl;
        const uint32_t kk = s1 ? k - segl : k;
        const float xr = s1 ? (p.y + (uint64_t)t * p.ldy)[kk]
                            : (p.embd ? embd_iq4(p.embd, (uint64_t)segl, p.embd_ne1, p.tok[t], kk)
                                      : (p.x + (uint64_t)t * p.ldx)[kk]);
        v = xr * (s1 ? p.w2 : p.w)[kk];
        ss = wave_sum64(xr * xr);
    } else if (RMS) {
        // x_eff = x + (p_0 + p_1 + ...) over the NP partial planes, written back to xnew;
        // v = x_eff * w, and the super-block's sum of x_eff^2 for the GEMV's row factor
        const float xr = KIND == ACT_RMS_EMBD ? embd_iq4(p.embd, (uint64_t)p.nsb * 256, p.embd_ne1, p.tok[t], k)
                                              : (p.x + (uint64_t)t * p.ldx)[k];
        float pr[NP > 0 ? NP : 1];
#pragma unroll
        for (int q = 0; q < NP; q++) pr[q] = (p.part + (uint64_t)q * p.pstride + (uint64_t)t * p.ldp)[k];
        const float wk = p.w[k];
        float xe = xr;
        if (NP > 0) {
            float ps = pr[0];
#pragma unroll
            for (int q = 1; q < NP; q++) ps += pr[q];
            xe += ps;
        }
        if (p.xnew) (p.xnew + (uint64_t)t * p.ldxn)[k] = xe;
        v = xe * wk;
        ss = wave_sum64(xe * xe);
    } else if (KIND == QGPU_ACT_GATED_NORM) {
        // heads of seg = 64 * hw elements: waves [h0, h0 + hw) of this block hold one head
        const int hw = (int)(p.seg >> 6), h0 = (wv / hw) * hw;
        const float raw = (p.x + (uint64_t)t * p.ldx)[k];
        const float gy = (p.y + (uint64_t)t * p.ldy)[k];
        const float wk = p.w[k & (uint32_t)(p.seg - 1)];
        const float sw = wave_sum64(raw * raw);
        if (lane == 0) ssw[wv] = sw;
        __syncthreads();
        float tot = ssw[h0];
        for (int q = 1; q < hw; q++) tot += ssw[h0 + q];
        const float sc = 1.0f / sqrtf(tot / (float)p.seg + p.eps);
        v = ((raw * sc) * wk) * silu_dev(gy);
    } else if (KIND == QGPU_ACT_SILU_MUL) {
        const float xv = (p.x + (uint64_t)t * p.ldx)[k];
        const float yv = (p.y + (uint64_t)t * p.ldy)[k];
        v = silu_dev(xv) * yv;
    } else {
        v = (p.x + (uint64_t)t * p.ldx)[k];
    }
    if (p.xout) (p.xout + (uint64_t)t * p.ldxo)[k] = v;
    const float mw = wave_max64(fabsf(v));
    if (lane == 0) {
        mxw[wv] = mw;
        if (RMS) ssw[wv] = ss;
    }
    __syncthreads();
    if (RMS && e == 0) p.rss[(uint64_t)t * p.nsb + sb] = (ssw[0] + ssw[1]) + (ssw[2] + ssw[3]);
    if (!p.digits) return;                                       // fp32 rows only (VALU formats)
    const float mx = fmaxf(fmaxf(mxw[0], mxw[1]), fmaxf(mxw[2], mxw[3]));
    tok_digits(v, mx, i, A + (uint64_t)a * PLANE_BYTES + (uint64_t)sb * DIGIT_TILE, xs + (uint64_t)a * XS_FLOATS + (uint64_t)sb * 16);
}

// ---------------------------------------------------------------- IQ4_XS MFMA GEMV
struct GemvMat {
    const uint8_t *W;
    float *out;
    uint64_t ldo;
    uint32_t rows, tile0, row_lo, row_hi;   // flat tile start; rows written: [row_lo, row_hi)
    uint32_t tile_first;                    // first tile of this matrix that is launched
    uint32_t blk0, ks;                      // first block; K ranges per tile (block q of a tile writes
    uint64_t pstride;                       // partial plane q at out + q * pstride when the launch splits)
};
struct GemvArgs {
    GemvMat m[QGPU_MAX_MULTI];
    int n_mat, nsb, ntok, flags;
    uint32_t pair0;                // IQ4_PAIR: flat tiles from pair0 on run as two half-K blocks each
    unsigned long long *xchg;      // IQ4_PAIR: their exchange slots, (tile - pair0) * PAIR_SLOTS + entry
    const uint8_t *A;
    const float *xs;
    const float *x;        // VALU path: fp32 activations
    uint64_t ldx, ne0;
    const float *rss;      // deferred RMSNorm: outputs *= 1/sqrt(sum_sb rss[t*rss_nsb+sb] * rss_inv_n + eps)
    int rss_nsb;
    float rss_inv_n, eps;
    int rss_seg;           // two segments (IQ4_RMS2): super-blocks [0, rss_seg) and [rss_seg, rss_nsb), each
                           // with its own factor (rss_inv_n = 1 / segment length)
};

// Row factors of the deferred RMSNorm, one per token, into rsc[]: wave w owns tokens
// w, w + nw, ... (NU = ceil(8 / nw) per wave); the per-super-block sums of squares are
// added in the same fixed order in every block.  rms_load issues the loads (before
// the main loop, so their latency is hidden), rms_reduce finishes after it.
// (rss_nsb <= 64: one sum per lane and token)
template <int NU> struct RmsPart { float v[NU]; };
template <int NU>
static __device__ __forceinline__ void rms_load(const GemvArgs &args, int wv, int nw, int lane, RmsPart<NU> &rp)
{
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int t = wv + u * nw;
        rp.v[u] = (t < args.ntok && lane < args.rss_nsb) ? args.rss[(uint64_t)t * args.rss_nsb + lane] : 0.0f;
    }
}
template <int NU>
static __device__ __forceinline__ void rms_reduce(const GemvArgs &args, int wv, int nw, int lane, const RmsPart<NU> &rp,
                                                  float *rsc)
{
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int t = wv + u * nw;
        const float s = wave_sum64(rp.v[u]);
        if (lane == 0 && t < args.ntok) rsc[t] = 1.0f / sqrtf(s * args.rss_inv_n + args.eps);
    }
}
// the same for two segments: rsc[t] from the sums of super-blocks [0, rss_seg), rsc1[t] from the rest
template <int NU>
static __device__ __forceinline__ void rms_reduce2(const GemvArgs &args, int wv, int nw, int lane,
                                                   const RmsPart<NU> &rp, float *rsc, float *rsc1)
{
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int t = wv + u * nw;
        const float s0 = wave_sum64(lane < args.rss_seg ? rp.v[u] : 0.0f);
        const float s1 = wave_sum64(lane < args.rss_seg ? 0.0f : rp.v[u]);
        if (lane == 0 && t < args.ntok) {
            rsc[t] = 1.0f / sqrtf(s0 * args.rss_inv_n + args.eps);
            rsc1[t] = 1.0f / sqrtf(s1 * args.rss_inv_n + args.eps);
        }
    }
}

// a * b + c on the low 24 bits of a and b (signed), 32-bit result.  Plain
// code, not inline asm: its input comes straight from an MFMA, and the
// compiler inserts the MFMA-to-VALU wait states only for instructions it
// generates itself.
#ifndef GEMV_MAD_SEP
#define GEMV_MAD_SEP 1
#endif
static __device__ __forceinline__ int mad24(int a, int b, int c)
{
    int r = __mul24(a, b) + c;
#if GEMV_MAD_SEP
    // an empty asm between the multiply-adds of a chain: the compiler otherwise
    // turns pairs of them into two multiplies and a v_add3_u32 (3 instructions
    // for 2 products instead of 2 v_mad_i32_i24)
    asm("" : "+v"(r));
#endif
    return r;
}

// Registers 0..2 of a lane's MFMA result are digits 0..2 of its token; register 3
// (digit slot 3) is always zero -- its A lanes load nothing -- so the scale and
// accumulate steps stop at DIGIT_REGS.
#ifndef DIGIT_REGS
#define DIGIT_REGS 3
#endif

// IQ4_NL codebook split across two 8-entry v_perm_b32 tables indexed by the
// whole nibble q: perm(XH:XL, q) + perm(YH:YL, q ^ 8) = c(q).  Selectors 8..15
// of v_perm_b32 give constants (8..11: sign of bytes 1, 3, 5, 7 as 0x00/0xFF;
// 12: 0x00; 13..15: 0xFF), so each table is exact for its own half and
// contributes 0 or -1 to the other, which the other table absorbs:
//   X = c(0..7) - {0, 0, 0, 0, 0, -1, -1, -1}   (Y bytes are positive)
//   Y = c(8..15) - {-1, -1, -1, -1, 0, -1, -1, -1} (X bytes are negative)
// The two halves are multiplied by the same activation operand in two chained
// MFMAs, so the integer dot product equals the one with the codebook bytes.
// 9 VALU operations per 8 weights (4 v_perm_b32).
static __device__ __forceinline__ void iq4_decode8(uint32_t q, uint32_t &x_lo, uint32_t &x_hi, uint32_t &y_lo,
                                                   uint32_t &y_hi)
{
    const uint32_t XL = 0xBFAD9881u, XH = 0xF7EBDECFu;      // -127 -104 -83 -65 | -49 -34 -21 -9
    const uint32_t YL = 0x271A0E02u, YH = 0x725A4635u;      //    2   14  26  39 |  53  70  90 114
    const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
    x_lo = __builtin_amdgcn_perm(XH, XL, lo);
    x_hi = __builtin_amdgcn_perm(XH, XL, hi);
    y_lo = __builtin_amdgcn_perm(YH, YL, lo ^ 0x08080808u);
    y_hi = __builtin_amdgcn_perm(YH, YL, hi ^ 0x08080808u);
}

// Weight records come from HBM and activation digits from L2, so the two are
// prefetched to different depths: weights IQ4_WDEPTH super-blocks ahead
// (10 VGPRs each), digits IQ4_ADEPTH1 / IQ4_ADEPTH2 ahead (16 * NA VGPRs each).
// Measured on MI355X: weights 2 ahead is 0.7% faster than 3 over the 27B step
// (decode 5.55 -> 5.49 ms), 4 ahead 5% slower.  Digits 2 ahead with one digit
// plane: 17408x5120 B = 4 15.0 -> 14.3 us, B = 1 14.7 -> 13.2 us, decode step
// 4.82 -> 4.70 ms, at 84 VGPRs (5 waves per SIMD instead of 7); with two planes
// 1-11% slower (B = 8 shapes), so those keep 1.
template <int FMT> struct WRec;                              // a lane's slice of one record
template <> struct WRec<T_IQ4_XS> { uint2 hdr; uint4 qa, qb; };
template <int NA>
struct IQ4A {
    uint4 av[NA][4];
    float4 xt[NA];       // 2^-s of tokens 0..3 of each plane (wave-uniform: scalar registers)
};

// rec, Ab, xsb are wave-uniform (scalar) addresses of this super-block's weight
// record, digit plane 0 and digit scales; lanes add their own offsets.  The A
// operand of lane l is digit l%4 of token (l%16)/4; lanes of digit 3 and of
// tokens past ntok load nothing (zero), and since each token's lanes read one
// 192-byte run per 768 bytes, a GEMV of B < 4 tokens reads about B/4 of the
// digit lines.  Result row
// 4 g + v of the matrix product (lane group g, register v) is digit v of token
// g: its scale is 2^(8 v) xs[g], from the four token scales (scalar loads).
// The digit loads are raw buffer loads over this super-block's tile: a lane of a
// token past ntok gets an offset beyond the record count, which reads zero and
// fetches nothing (no branch around the loads).
#define DIGIT_OOB 0x80000000u
#define DIGIT_RECORDS 0x40000000          // > NA planes of the workspace; < DIGIT_OOB
template <int NA>
static __device__ __forceinline__ void iq4_load_a(IQ4A<NA> &x, const uint8_t *Ab, const float *xsb, int lane,
                                                  int ntok)
{
    const int tk = (lane & 15) >> 2, dg = lane & 3;
    const uint32_t off = (uint32_t)(tk * 12 + (lane >> 4) * 3 + dg) * 16;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)Ab, 0, DIGIT_RECORDS, 0x00020000);
#pragma unroll
    for (int a = 0; a < NA; a++) {
        const uint32_t vo = dg < 3 && 4 * a + tk < ntok ? (uint32_t)(a * PLANE_BYTES) + off : DIGIT_OOB;
#pragma unroll
        for (int p = 0; p < 4; p++)
            x.av[a][p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, vo + p * DIGIT_SUB, 0, 0));
        x.xt[a] = *(const float4 *)(xsb + (uint64_t)a * XS_FLOATS);
    }
}

// 2^(8 v): the weight of digit v
static __device__ __forceinline__ float p8(int v) { return __builtin_bit_cast(float, (uint32_t)(127 + 8 * v) << 23); }
// scale of token g (this lane group's) from the four token scales
// (oh: the one-hot of the lane group, so the choice is four exact multiply-adds with the
// scales as scalar operands, not a branch per lane group)
static __device__ __forceinline__ float tok_scale(float4 xt, const float4 &oh)
{
    return fmaf(xt.w, oh.w, fmaf(xt.z, oh.z, fmaf(xt.y, oh.y, xt.x * oh.x)));
}

template <int NA>
static __device__ __forceinline__ void iq4_compute(const WRec<T_IQ4_XS> &w, const IQ4A<NA> &x, const float4 &g, float (&accf)[NA][4])
{
    const uint32_t qd[8] = { w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w };
    v4i acci[NA];
#pragma unroll
    for (int a = 0; a < NA; a++) acci[a] = (v4i){0, 0, 0, 0};
#pragma unroll
    for (int ib = 0; ib < 8; ib++) {
        uint32_t x_lo, x_hi, y_lo, y_hi;
        iq4_decode8(qd[ib], x_lo, x_hi, y_lo, y_hi);
        const long bx = (long)(((uint64_t)x_hi << 32) | x_lo), by = (long)(((uint64_t)y_hi << 32) | y_lo);
        const int wsc = hdr_scale(w.hdr, ib);
#pragma unroll
        for (int a = 0; a < NA; a++) {
            const uint4 q4 = x.av[a][ib >> 1];
            const long aop = (ib & 1) ? (long)(((uint64_t)q4.w << 32) | q4.z)
                                      : (long)(((uint64_t)q4.y << 32) | q4.x);
            const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                aop, by, __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bx, (v4i){0, 0, 0, 0}, 0, 0, 0), 0, 0, 0);
            // |D| < 2^19, |wsc| <= 32: exact 24-bit multiply-add
#pragma unroll
            for (int i = 0; i < DIGIT_REGS; i++) acci[a][i] = mad24(D[i], wsc, acci[a][i]);
        }
    }
    const float d = h2f(w.hdr.x & 0xFFFFu);
#pragma unroll
    for (int a = 0; a < NA; a++) {
        const float dx = d * tok_scale(x.xt[a], g);     // digit v's weight 2^(8 v) is applied at the end
#pragma unroll
        for (int v = 0; v < DIGIT_REGS; v++) accf[a][v] += (float)acci[a][v] * dx;
    }
}

// ---- K-quant and Q8_0 records on the same int8 matrix-core path.  A lane's
// slice of one record (see the record layouts above), then the per-sub-block
// work: the integer B operand (0..15 / 0..31 / 0..63 / int8 bytes), the exact
// int32 sub-block products, the scales.
//   Q4_K, Q5_K: sum_ib sc_ib D_ib in int32 (24-bit products, as IQ4_XS) and the
//     min term sum_ib m_ib (sum of the sub-block's activations) in the matrix
//     core itself: a second MFMA chain whose B operand is m_ib in every K slot;
//     output d * first - dmin * second.
//   Q6_K: two scale groups of 16 per sub-block = the lane's two dwords (elements
//     4g+c in 0..15, 16+4g+c in 16..31): one MFMA per group with the other
//     dword zero, and the -32 offset of the 6-bit values as one more chained
//     MFMA with the constant byte -32.
//   Q8_0: int8 quants as they are; the fp16 scale of each 32-element block in fp32.
template <> struct WRec<T_Q4_K> { uint4 hdr; uint4 qa, qb; };
template <> struct WRec<T_Q5_K> { uint4 hdr; uint4 qa, qb; uint2 hb; };
template <> struct WRec<T_Q6_K> { uint4 sc; uint4 qa, qb; uint4 hb; uint32_t d; };
template <> struct WRec<T_Q8_0> { uint4 hdr; uint4 q[4]; };

template <int FMT>
static __device__ __forceinline__ void kq_load_w(WRec<FMT> &w, const uint8_t *rec, int lane, int n)
{
    if constexpr (FMT == T_IQ4_XS) {
        w.hdr = *(const uint2 *)(rec + n * 8);
        w.qa = *(const uint4 *)(rec + IQ4_HDR_BYTES + lane * 16);
        w.qb = *(const uint4 *)(rec + IQ4_HDR_BYTES + 1024 + lane * 16);
    } else if constexpr (FMT == T_Q8_0) {
        w.hdr = *(const uint4 *)(rec + n * 16);
#pragma unroll
        for (int p = 0; p < 4; p++) w.q[p] = *(const uint4 *)(rec + KQ_Q + (p * 64 + lane) * 16);
    } else if constexpr (FMT == T_Q6_K) {
        w.sc = *(const uint4 *)(rec + n * 16);
        w.d = *(const uint16_t *)(rec + KQ_D6 + 2 * n);
        w.qa = *(const uint4 *)(rec + KQ_Q6 + lane * 16);
        w.qb = *(const uint4 *)(rec + KQ_Q6 + 1024 + lane * 16);
        w.hb = *(const uint4 *)(rec + KQ_HB6 + lane * 16);
    } else {
        w.hdr = *(const uint4 *)(rec + n * 16);
        w.qa = *(const uint4 *)(rec + KQ_Q + lane * 16);
        w.qb = *(const uint4 *)(rec + KQ_Q + 1024 + lane * 16);
        if constexpr (FMT == T_Q5_K) w.hb = *(const uint2 *)(rec + KQ_HB5 + lane * 8);
    }
}

static __device__ __forceinline__ uint32_t u4_get(uint4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
// bit c (c < 4) of x to bit 0 of byte c
static __device__ __forceinline__ uint32_t spread4(uint32_t x) { return (x * 0x00204081u) & 0x01010101u; }

template <int NA>
static __device__ __forceinline__ long kq_aop(const IQ4A<NA> &x, int a, int ib)
{
    const uint4 q4 = x.av[a][ib >> 1];
    return (ib & 1) ? (long)(((uint64_t)q4.w << 32) | q4.z) : (long)(((uint64_t)q4.y << 32) | q4.x);
}
static __device__ __forceinline__ long kq_b(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

template <int FMT, int NA>
static __device__ __forceinline__ void kq_compute(const WRec<FMT> &w, const IQ4A<NA> &x, const float4 &g, float (&accf)[NA][4])
{
    const v4i z4 = (v4i){0, 0, 0, 0};
    if constexpr (FMT == T_Q8_0) {
        float accs[NA][4];
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int i = 0; i < DIGIT_REGS; i++) accs[a][i] = 0.0f;
#pragma unroll
        for (int ib = 0; ib < 8; ib++) {
            const uint4 q = w.q[ib >> 1];
            const long b = (ib & 1) ? kq_b(q.z, q.w) : kq_b(q.x, q.y);
            const float dib = h2f((u4_get(w.hdr, ib >> 1) >> (16 * (ib & 1))) & 0xFFFFu);
#pragma unroll
            for (int a = 0; a < NA; a++) {
                const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(kq_aop<NA>(x, a, ib), b, z4, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < DIGIT_REGS; i++) accs[a][i] = fmaf((float)D[i], dib, accs[a][i]);
            }
        }
#pragma unroll
        for (int a = 0; a < NA; a++) {
            const float xg = tok_scale(x.xt[a], g);
#pragma unroll
            for (int v = 0; v < DIGIT_REGS; v++) accf[a][v] += accs[a][v] * xg;
        }
    } else if constexpr (FMT == T_Q6_K) {
        const uint32_t qd[8] = { w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w };
        const uint32_t NEG32 = 0xE0E0E0E0u;                     // int8 -32 in every byte
        v4i acc[NA];
#pragma unroll
        for (int a = 0; a < NA; a++) acc[a] = z4;
#pragma unroll
        for (int ib = 0; ib < 8; ib++) {
            const uint32_t hw = u4_get(w.hb, ib >> 1) >> (4 * (ib & 1));
            const uint32_t lo = (qd[ib] & 0x0F0F0F0Fu) | ((hw << 4) & 0x30303030u);
            const uint32_t hi = ((qd[ib] >> 4) & 0x0F0F0F0Fu) | ((hw << 2) & 0x30303030u);
            const uint32_t scw = u4_get(w.sc, ib >> 1);
            const int sa = (int)(int8_t)((scw >> (16 * (ib & 1))) & 0xFF), sb2 = (int)(int8_t)((scw >> (16 * (ib & 1) + 8)) & 0xFF);
#pragma unroll
            for (int a = 0; a < NA; a++) {
                const long aop = kq_aop<NA>(x, a, ib);
                const v4i DA = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                    aop, kq_b(lo, 0), __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, kq_b(NEG32, 0), z4, 0, 0, 0), 0, 0, 0);
                const v4i DB = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                    aop, kq_b(0, hi), __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, kq_b(0, NEG32), z4, 0, 0, 0), 0, 0, 0);
#pragma unroll
                for (int i = 0; i < DIGIT_REGS; i++) acc[a][i] = mad24(DA[i], sa, mad24(DB[i], sb2, acc[a][i]));
            }
        }
        const float d = h2f(w.d & 0xFFFFu);
#pragma unroll
        for (int a = 0; a < NA; a++) {
            const float dx = d * tok_scale(x.xt[a], g);
#pragma unroll
            for (int v = 0; v < DIGIT_REGS; v++) accf[a][v] += (float)acc[a][v] * dx;
        }
    } else {                                                   // Q4_K, Q5_K
        const uint32_t qd[8] = { w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w };
        v4i acq[NA], acm[NA];
#pragma unroll
        for (int a = 0; a < NA; a++) { acq[a] = z4; acm[a] = z4; }
#pragma unroll
        for (int ib = 0; ib < 8; ib++) {
            uint32_t lo = qd[ib] & 0x0F0F0F0Fu, hi = (qd[ib] >> 4) & 0x0F0F0F0Fu;
            if constexpr (FMT == T_Q5_K) {
                const uint32_t hbb = ((ib < 4 ? w.hb.x : w.hb.y) >> (8 * (ib & 3))) & 0xFFu;
                lo |= spread4(hbb & 15u) << 4;
                hi |= spread4(hbb >> 4) << 4;
            }
            const int sc = (int)kq_sc(w.hdr, ib);
            const uint32_t mrep = kq_m(w.hdr, ib) * 0x01010101u;
#pragma unroll
            for (int a = 0; a < NA; a++) {
                const long aop = kq_aop<NA>(x, a, ib);
                const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, kq_b(lo, hi), z4, 0, 0, 0);
                acm[a] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, kq_b(mrep, mrep), acm[a], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < DIGIT_REGS; i++) acq[a][i] = mad24(D[i], sc, acq[a][i]);
            }
        }
        const float d = h2f(w.hdr.x & 0xFFFFu), dm = h2f(w.hdr.x >> 16);
#pragma unroll
        for (int a = 0; a < NA; a++) {
            const float xg = tok_scale(x.xt[a], g), dx = d * xg, dmx = dm * xg;
#pragma unroll
            for (int v = 0; v < DIGIT_REGS; v++)
                accf[a][v] += (float)acq[a][v] * dx - (float)acm[a][v] * dmx;
        }
    }
}

#ifndef IQ4_WDEPTH
#define IQ4_WDEPTH 2    // weight records in flight per wave
#endif
#ifndef IQ4_ADEPTH1
#define IQ4_ADEPTH1 2   // digit super-blocks in flight per wave, one digit plane (B <= 4)
#endif
#ifndef IQ4_ADEPTH2
#define IQ4_ADEPTH2 1   // the same, two digit planes (B = 5..8: 20 more VGPRs per slot)
#endif

// MODE bit 0 (IQ4_RMS): deferred RMSNorm row factors; bit 1 (IQ4_SPLIT): K split
// into partial planes.  Plain launches (MODE 0) compile without either.
#define IQ4_RMS   1
#define IQ4_SPLIT 2
#define IQ4_PAIR  4     // tail balance: the last tiles of the launch in two K halves (never with IQ4_SPLIT)
#define IQ4_NORING 16   // no prefetch rings: each step loads its weight record and digits at the step
                        // (IQ4_XS, one digit plane, 3 or 4 waves per tile; see launch_group)
#define IQ4_RMS2  8     // deferred two-segment RMSNorm: each segment's super-blocks are summed apart (a wave
                        // meets its second-segment super-blocks after all its first-segment ones, so its
                        // sums move aside once), and each sum takes its segment's row factor (never with
                        // IQ4_RMS or IQ4_SPLIT)
template <int FMT, int NA, int NW, int MODE>
#ifndef IQ4_MINW1
#define IQ4_MINW1 1     // minimum waves per SIMD the compiler must allow (caps VGPRs), one digit plane
#endif
#ifndef IQ4_MINW2
#define IQ4_MINW2 1     // the same, two digit planes
#endif
__global__ __launch_bounds__(NW * 64, NA == 1 ? IQ4_MINW1 : IQ4_MINW2) void k_gemv_mfma(const GemvArgs args)
{
    constexpr bool SEG2 = (MODE & IQ4_RMS2) != 0;
    __shared__ float red[NW][NA][4][16];
    __shared__ float red1[SEG2 ? NW : 1][NA][4][16];        // the second segment's sums
    __shared__ float rsc[QGPU_MAX_B], rsc1[SEG2 ? QGPU_MAX_B : 1];
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const float4 oh = make_float4(g == 0, g == 1, g == 2, g == 3);   // token g of this lane group
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);     // wave-uniform: scalar loop control
    int k = 0;
    uint32_t T;                    // row tile of this block within its matrix
    int ks = 1, kq = 0;            // K ranges of the tile, and this block's
    uint32_t pflat = 0;            // IQ4_PAIR: flat tile index
    if (MODE & IQ4_PAIR) {
        const uint32_t u = blockIdx.x >= args.pair0 ? blockIdx.x - args.pair0 : 0;
        pflat = blockIdx.x < args.pair0 ? blockIdx.x : args.pair0 + (u >> 1);
        if (blockIdx.x >= args.pair0) { ks = 2; kq = (int)(u & 1); }
        while (k + 1 < args.n_mat && pflat >= args.m[k + 1].tile0) k++;
        T = pflat - args.m[k].tile0 + args.m[k].tile_first;
    } else {
        while (k + 1 < args.n_mat && blockIdx.x >= args.m[k + 1].blk0) k++;
        const uint32_t lb = blockIdx.x - args.m[k].blk0;            // block within matrix k
        if (MODE & IQ4_SPLIT) { ks = (int)args.m[k].ks; kq = (int)(lb % (uint32_t)ks); }
        T = ((MODE & IQ4_SPLIT) ? lb / (uint32_t)ks : lb) + args.m[k].tile_first;
    }
    const GemvMat &M = args.m[k];
    const int nsb = args.nsb;
    constexpr uint32_t REC = FMT == T_IQ4_XS ? IQ4_REC_BYTES : FMT == T_Q4_K ? 2304 : FMT == T_Q5_K ? 2816 : FMT == T_Q6_K ? 3360 : 4352;
    const uint8_t *rec0 = M.W + (uint64_t)T * nsb * REC;
    const int kb0 = kq * nsb / ks, nkb = (kq + 1) * nsb / ks - kb0;
    // wave wv takes super-blocks kb0 + wv, kb0 + wv + NW, ... of the block's K range: the waves of a
    // compute unit then read neighbouring digit tiles at about the same time (steps j = 0..nsw-1;
    // 17408x5120 B = 4 13.78 -> 13.56 us against contiguous quarters)
    const int nsw = wv < nkb ? (nkb - wv + NW - 1) / NW : 0;
#define SBX(j) (kb0 + wv + (j) * NW)
    const bool seg1_last = SEG2 && nsw > 0 && SBX(nsw - 1) >= args.rss_seg;   // the wave ends in the second segment
    RmsPart<(QGPU_MAX_B + NW - 1) / NW> rp;
    if (MODE & (IQ4_RMS | IQ4_RMS2)) rms_load(args, wv, NW, lane, rp);

    float accf[NA][4], accf0[NA][4];                     // accf0: the first segment's sums (SEG2 only)
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int i = 0; i < 4; i++) accf[a][i] = 0.0f;
    if constexpr (SEG2)
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int i = 0; i < 4; i++) accf0[a][i] = 0.0f;

    // two register rings: each step issues the loads of step j+WDEPTH-1 (weights) and
    // j+ADEPTH-1 (digits) before step j is decoded and multiplied (ring indices are
    // compile-time after unrolling by UNROLL); digit loads before weight loads.  The
    // loads of the last steps are skipped by a branch, so the compiler's waits also
    // cover the newest loads (vmcnt(1), then vmcnt(0) within the step): in effect a
    // wave has about one step's records in flight.  IQ4_NORING: depth 1.
    constexpr bool RING = !(MODE & IQ4_NORING);
    constexpr int WDEPTH = RING ? IQ4_WDEPTH : 1;
    constexpr int ADEPTH = RING ? (NA == 1 ? IQ4_ADEPTH1 : IQ4_ADEPTH2) : 1;
    // main-loop unroll: a common multiple of the two ring depths (compile-time ring slots)
    constexpr int UNROLL = (WDEPTH % ADEPTH) == 0 ? WDEPTH : WDEPTH * ADEPTH;
    WRec<FMT> wr[WDEPTH];
    IQ4A<NA> ar[ADEPTH];
#define LOAD_W(slot, j) kq_load_w<FMT>(wr[slot], rec0 + (uint64_t)SBX(j) * REC, lane, n)
#define LOAD_A(slot, j) iq4_load_a<NA>(ar[slot], args.A + (uint64_t)SBX(j) * DIGIT_TILE, args.xs + (uint64_t)SBX(j) * 16, lane, args.ntok)
#pragma unroll
    for (int d = 0; d < WDEPTH - 1 || d < ADEPTH - 1; d++) {
        if (d < ADEPTH - 1 && d < nsw) LOAD_A(d, d);
        if (d < WDEPTH - 1 && d < nsw) LOAD_W(d, d);
    }
    for (int j = 0; j < nsw; j += UNROLL) {
#pragma unroll
        for (int d = 0; d < UNROLL; d++) {
            if (j + d < nsw) {
                const int pw = j + d + WDEPTH - 1, pa = j + d + ADEPTH - 1;
                if (pa < nsw) LOAD_A((d + ADEPTH - 1) % ADEPTH, pa);
                if (pw < nsw) LOAD_W((d + WDEPTH - 1) % WDEPTH, pw);
                if (SEG2 && SBX(j + d) >= args.rss_seg && SBX(j + d) - NW < args.rss_seg) {
                    // this wave's first super-block of the second segment (wave-uniform, once)
#pragma unroll
                    for (int a = 0; a < NA; a++)
#pragma unroll
                        for (int i = 0; i < 4; i++) { accf0[a][i] = accf[a][i]; accf[a][i] = 0.0f; }
                }
                if constexpr (FMT == T_IQ4_XS) iq4_compute<NA>(wr[d % WDEPTH], ar[d % ADEPTH], oh, accf);
                else kq_compute<FMT, NA>(wr[d % WDEPTH], ar[d % ADEPTH], oh, accf);
            }
        }
    }
#undef LOAD_W
#undef LOAD_A
#undef SBX
    if (MODE & IQ4_RMS) rms_reduce(args, wv, NW, lane, rp, rsc);
    if constexpr (SEG2) {
        rms_reduce2(args, wv, NW, lane, rp, rsc, rsc1);
        // the wave's sums of each segment: its second-segment super-blocks, if any, came last
        if (seg1_last) {
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int i = 0; i < 4; i++) { const float f1 = accf[a][i]; accf[a][i] = accf0[a][i]; accf0[a][i] = f1; }
        } else {
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int i = 0; i < 4; i++) accf0[a][i] = 0.0f;
        }
    }
    // registers 0..3 of lane (g, n) hold digits 0..3 of token g, row n: sum them with their weights
    // 2^(8 v) (a power of two: the same bits as weighting every super-block's term); SEG2: accf the
    // first segment's sums, accf0 the second's
#pragma unroll
    for (int a = 0; a < NA; a++) {
        red[wv][a][g][n] = DIGIT_REGS == 3 ? (accf[a][0] + accf[a][1] * p8(1)) + accf[a][2] * p8(2)
                                           : (accf[a][0] + accf[a][1] * p8(1)) + (accf[a][2] * p8(2) + accf[a][3] * p8(3));
        if constexpr (SEG2)
            red1[wv][a][g][n] = DIGIT_REGS == 3 ? (accf0[a][0] + accf0[a][1] * p8(1)) + accf0[a][2] * p8(2)
                                                : (accf0[a][0] + accf0[a][1] * p8(1)) + (accf0[a][2] * p8(2) + accf0[a][3] * p8(3));
    }
    __syncthreads();
    for (int e = tid; e < NA * 64; e += NW * 64) {     // (plane, token, row) entries of the tile
        const int a = e >> 6, i = (e >> 4) & 3, nn = e & 15;
        float s = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) s += red[w][a][i][nn];
        if constexpr (SEG2)
#pragma unroll
            for (int w = 0; w < NW; w++) s1 += red1[w][a][i][nn];
        const int t = 4 * a + i;
        const uint32_t r = T * IQ4_TILE_ROWS + nn;
        if (t < args.ntok && r >= M.row_lo && r < M.row_hi) {
            if (MODE & IQ4_RMS) s *= rsc[t];
            if constexpr (SEG2) s = s * rsc[t] + s1 * rsc1[t];
            if ((MODE & IQ4_PAIR) && ks == 2) {
                // two contributors per entry: the first leaves its half in the slot, the second
                // takes it (the exchange itself carries the value, so no fence), writes the sum and
                // clears the slot.  a + b and b + a are the same bits, whichever half comes first.
                unsigned long long *slot = args.xchg + (uint64_t)(pflat - args.pair0) * PAIR_SLOTS + e;
                const unsigned long long old =
                    atomicExch(slot, (1ull << 32) | (unsigned long long)__float_as_uint(s));
                if (old >> 32) {
                    s = __uint_as_float((uint32_t)old) + s;
                    atomicExch(slot, 0ull);
                    float *o = M.out + (uint64_t)t * M.ldo + r;
                    *o = (args.flags & QGPU_GEMV_ACCUM) ? *o + s : s;
                }
            } else if (MODE & IQ4_SPLIT) {
                M.out[(uint64_t)kq * M.pstride + (uint64_t)t * M.ldo + r] = s;
            } else {
                float *o = M.out + (uint64_t)t * M.ldo + r;
                *o = (args.flags & QGPU_GEMV_ACCUM) ? *o + s : s;
            }
        }
    }
}

// ---------------------------------------------------------------- wide GEMV (activations in LDS)
// For a matrix of many tiles and a short K (the 248,320-row lm_head: 15,520 tiles, K = 5120), the
// kernel above re-reads the digit tile of every (tile, super-block) from L2: 3 KB per 2.2 KB weight
// record at B = 4 (931 MB of digits against 675 MB of weights per call).  Here a block copies the
// call's digit planes into LDS once (NA x nsb x 3 KB) and each of its waves streams whole
// tiles (every super-block of a tile in order), tile after tile (tiles wave0, wave0 + waves of the
// grid, ...), its weight ring running on across tile ends; the A operand comes from LDS, one
// super-block ahead.  A wave owns its tile's outputs, so there is no cross-wave reduction.  The
// A rows of digit slot 3 and of tokens past ntok read whatever the tile holds there: their
// products land in result register 3 (never used) and in the lane groups of those tokens (never
// written).  Single matrix, no K split; the deferred RMSNorm row factor as in k_gemv_mfma.
// One block per compute unit, of as many waves as the kernel's VGPRs let each SIMD hold: one digit
// plane 16 (IQ4_XS..Q6_K, 100-128 VGPRs) or 12 (Q8_0, 144); two planes 12 (IQ4_XS, Q4_K: 155-166)
// or 8 (the others, which would spill at 12).  (Two blocks of 10 waves with one plane: 4 waves per
// SIMD by the VGPR granule, so 10 per compute unit, measured 17% slower.)
#define WIDE_BPC(NA) 1
#define WIDE_NW(FMT, NA) ((NA) == 1 ? ((FMT) == T_Q8_0 ? 12 : 16) : ((FMT) == T_IQ4_XS || (FMT) == T_Q4_K ? 12 : 8))
#define WIDE_NSB(NA) 20                      // super-blocks the LDS operand holds (K <= 5120): NA x 60 KB
#ifndef WIDE_WDEPTH
#define WIDE_WDEPTH 3       // weight records in flight per wave
#endif
template <int NA>
static __device__ __forceinline__ void lds_load_a(IQ4A<NA> &x, const uint8_t *dig, uint32_t pbytes, int sb,
                                                  const float *xs, int lane)
{
    const int tk = (lane & 15) >> 2, dg = lane & 3;
    const uint32_t off = (uint32_t)sb * DIGIT_TILE + (uint32_t)(tk * 12 + (lane >> 4) * 3 + (dg < 3 ? dg : 2)) * 16;
#pragma unroll
    for (int a = 0; a < NA; a++) {
#pragma unroll
        for (int p = 0; p < 4; p++) x.av[a][p] = *(const uint4 *)(dig + (uint32_t)a * pbytes + off + p * DIGIT_SUB);
        x.xt[a] = *(const float4 *)(xs + (uint64_t)a * XS_FLOATS + (uint64_t)sb * 16);
    }
}

template <int FMT, int NA, int MODE>
__global__ __launch_bounds__(WIDE_NW(FMT, NA) * 64) void k_gemv_wide(const GemvArgs args)
{
    constexpr int NWW = WIDE_NW(FMT, NA);
    __shared__ __attribute__((aligned(16))) uint8_t dig[NA * WIDE_NSB(NA) * DIGIT_TILE];
    __shared__ float rsc[QGPU_MAX_B];
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const float4 oh = make_float4(g == 0, g == 1, g == 2, g == 3);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const GemvMat &M = args.m[0];
    const int nsb = args.nsb;
    const uint32_t ntiles = args.pair0, stride = gridDim.x * NWW;           // tiles of the launch
    constexpr uint32_t REC = FMT == T_IQ4_XS ? IQ4_REC_BYTES : FMT == T_Q4_K ? 2304 : FMT == T_Q5_K ? 2816 : FMT == T_Q6_K ? 3360 : 4352;
    const uint32_t t0 = blockIdx.x * NWW + wv;
    const int nst = t0 < ntiles ? (int)((ntiles - 1 - t0) / stride + 1) * nsb : 0;    // this wave's steps
    const uint8_t *W0 = M.W + (uint64_t)M.tile_first * nsb * REC;
    // weight cursor (tile, super-block) of the next record to load; the first records go out
    // before the LDS copy
    uint32_t lt = t0;
    int lsb = 0;
    WRec<FMT> wr[WIDE_WDEPTH];
#define WIDE_ADV(t_, sb_) do { if (++(sb_) == nsb) { (sb_) = 0; (t_) += stride; } } while (0)
#define WIDE_LOAD_W(slot) do { kq_load_w<FMT>(wr[slot], W0 + ((uint64_t)lt * nsb + lsb) * REC, lane, n); \
                               WIDE_ADV(lt, lsb); } while (0)
#pragma unroll
    for (int d = 0; d < WIDE_WDEPTH - 1; d++)
        if (d < nst) WIDE_LOAD_W(d);
    RmsPart<(QGPU_MAX_B + NWW - 1) / NWW> rp;
    if (MODE & IQ4_RMS) rms_load(args, wv, NWW, lane, rp);
    const uint32_t pbytes = (uint32_t)nsb * DIGIT_TILE;
    for (uint32_t i = (uint32_t)tid * 16u; i < NA * pbytes; i += NWW * 64 * 16) {
        const uint32_t a = i >= pbytes ? 1u : 0u, o = i - a * pbytes;
        *(uint4 *)(dig + i) = *(const uint4 *)(args.A + (uint64_t)a * PLANE_BYTES + o);
    }
    if (MODE & IQ4_RMS) rms_reduce(args, wv, NWW, lane, rp, rsc);
    __syncthreads();

    float accf[NA][4];
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int i = 0; i < 4; i++) accf[a][i] = 0.0f;
    uint32_t ct = t0;          // compute cursor
    int csb = 0;
    IQ4A<NA> ar[2];
    if (nst > 0) lds_load_a<NA>(ar[0], dig, pbytes, 0, args.xs, lane);
    // ring slots are compile-time after unrolling by a common multiple of the two depths
    constexpr int UNROLL = WIDE_WDEPTH % 2 == 0 ? WIDE_WDEPTH : 2 * WIDE_WDEPTH;
    for (int j = 0; j < nst; j += UNROLL) {
#pragma unroll
        for (int d = 0; d < UNROLL; d++) {
            if (j + d < nst) {
                if (j + d + WIDE_WDEPTH - 1 < nst) WIDE_LOAD_W((d + WIDE_WDEPTH - 1) % WIDE_WDEPTH);
                if (j + d + 1 < nst) lds_load_a<NA>(ar[(d + 1) & 1], dig, pbytes, csb + 1 < nsb ? csb + 1 : 0, args.xs, lane);
                if constexpr (FMT == T_IQ4_XS) iq4_compute<NA>(wr[d % WIDE_WDEPTH], ar[d & 1], oh, accf);
                else kq_compute<FMT, NA>(wr[d % WIDE_WDEPTH], ar[d & 1], oh, accf);
                if (csb == nsb - 1) {                      // the tile's last super-block: its outputs
                    const uint32_t r = (M.tile_first + ct) * IQ4_TILE_ROWS + n;
#pragma unroll
                    for (int a = 0; a < NA; a++) {
                        const int t = 4 * a + g;
                        float s = DIGIT_REGS == 3 ? (accf[a][0] + accf[a][1] * p8(1)) + accf[a][2] * p8(2)
                                                  : (accf[a][0] + accf[a][1] * p8(1)) + (accf[a][2] * p8(2) + accf[a][3] * p8(3));
                        if (t < args.ntok && r >= M.row_lo && r < M.row_hi) {
                            if (MODE & IQ4_RMS) s *= rsc[t];
                            float *o = M.out + (uint64_t)t * M.ldo + r;
                            *o = (args.flags & QGPU_GEMV_ACCUM) ? *o + s : s;
                        }
#pragma unroll
                        for (int i = 0; i < 4; i++) accf[a][i] = 0.0f;
                    }
                }
                WIDE_ADV(ct, csb);
            }
        }
    }
#undef WIDE_LOAD_W
#undef WIDE_ADV
}

// ---------------------------------------------------------------- VALU GEMV (GGUF layout)
// Decoders of one 32-element chunk to the dequantised fp32 values (bit-exact
// with the scalar reference: explicit round-to-nearest products, no FMA).
static __device__ __forceinline__ uint32_t ld8(const uint8_t *p) { return *p; }

template <int FMT>
static __device__ __forceinline__ void decode_chunk(const uint8_t *__restrict__ row, uint32_t c, float w[32])
{
    if (FMT == T_F32) {
        const float4 *p = (const float4 *)(row + (uint64_t)c * 128);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 v = p[j];
            w[4 * j] = v.x; w[4 * j + 1] = v.y; w[4 * j + 2] = v.z; w[4 * j + 3] = v.w;
        }
    } else if (FMT == T_Q8_0) {
        const uint8_t *b = row + (uint64_t)c * 34;
        const float d = h2f(ld8(b) | (ld8(b + 1) << 8));
#pragma unroll
        for (int j = 0; j < 32; j++) w[j] = __fmul_rn(d, (float)(int8_t)b[2 + j]);
    } else if (FMT == T_Q4_K || FMT == T_Q5_K) {
        const uint32_t sbi = c >> 3, j = c & 7, g = j >> 1, half = j & 1;
        const uint8_t *b = row + (uint64_t)sbi * (FMT == T_Q5_K ? 176 : 144);
        const float d = h2f(*(const uint16_t *)b), dmin = h2f(*(const uint16_t *)(b + 2));
        const uint8_t *sc = b + 4;
        uint32_t s, m;
        if (j < 4) { s = sc[j] & 63; m = sc[j + 4] & 63; }
        else { s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4); m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4); }
        const float d1 = __fmul_rn(d, (float)s), m1 = __fmul_rn(dmin, (float)m);
        const uint8_t *qs = b + (FMT == T_Q5_K ? 48 : 16) + 32 * g;
        const uint4 q0 = ((const uint4 *)qs)[0], q1 = ((const uint4 *)qs)[1];
        const uint32_t qw[8] = { q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w };
        uint32_t hw[8];
        if (FMT == T_Q5_K) {
            const uint4 h0 = ((const uint4 *)(b + 16))[0], h1 = ((const uint4 *)(b + 16))[1];
            hw[0] = h0.x; hw[1] = h0.y; hw[2] = h0.z; hw[3] = h0.w; hw[4] = h1.x; hw[5] = h1.y; hw[6] = h1.z; hw[7] = h1.w;
        }
        const uint32_t hb = 2 * g + half;
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t byte = (qw[l >> 2] >> (8 * (l & 3))) & 0xFF;
            uint32_t q = half ? (byte >> 4) : (byte & 15);
            if (FMT == T_Q5_K) q += ((((hw[l >> 2] >> (8 * (l & 3))) & 0xFF) >> hb) & 1) << 4;
            w[l] = __fsub_rn(__fmul_rn(d1, (float)q), m1);
        }
    } else if (FMT == T_Q6_K) {
        const uint32_t sbi = c >> 3, j = c & 7, nh = j >> 2, quad = j & 3;
        const uint8_t *b = row + (uint64_t)sbi * 210;
        const float d = h2f(ld8(b + 208) | (ld8(b + 209) << 8));
        const uint8_t *ql = b + 64 * nh + ((quad & 1) ? 32 : 0), *qh = b + 128 + 32 * nh;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * nh);
        const float ds0 = __fmul_rn(d, (float)sc[2 * quad]), ds1 = __fmul_rn(d, (float)sc[2 * quad + 1]);
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t lo = ql[l];
            const uint32_t nib = (quad & 2) ? (lo >> 4) : (lo & 15);
            const int q = (int)(nib | (((qh[l] >> (2 * quad)) & 3) << 4)) - 32;
            w[l] = __fmul_rn(l < 16 ? ds0 : ds1, (float)q);
        }
    }
}

// one wave per 2 rows, lanes stride over 32-element chunks (F32: over elements); 4 waves per block
template <int FMT, int NT>
__global__ __launch_bounds__(256) void k_gemv_valu(const GemvArgs args)
{
    __shared__ float rsc[QGPU_MAX_B];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (args.rss) {
        RmsPart<2> rp;
        rms_load(args, wv, 4, lane, rp);
        rms_reduce(args, wv, 4, lane, rp, rsc);
        __syncthreads();
    }
    const uint32_t grp = blockIdx.x;                  // flat row-group (8 rows) index
    int k = 0;
    while (k + 1 < args.n_mat && grp >= args.m[k + 1].tile0) k++;
    const GemvMat &M = args.m[k];
    const uint32_t r0 = (grp - M.tile0 + M.tile_first) * 8 + wv * 2;
    const uint64_t rb = (FMT == T_F32) ? args.ne0 * 4 : (FMT == T_Q8_0 ? args.ne0 / 32 * 34 :
                        args.ne0 / 256 * (FMT == T_Q4_K ? 144 : FMT == T_Q5_K ? 176 : 210));
    const int nr = (r0 >= M.row_hi) ? 0 : (r0 + 1 >= M.row_hi ? 1 : 2);
    float acc[2][NT];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = 0.0f;
    if (FMT == T_F32) {
        for (uint64_t i = lane; i < args.ne0; i += 64) {
            float w[2];
            for (int r = 0; r < 2; r++) w[r] = r < nr ? ((const float *)(M.W + (uint64_t)(r0 + r) * rb))[i] : 0.0f;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float xv = t < args.ntok ? args.x[(uint64_t)t * args.ldx + i] : 0.0f;
                acc[0][t] = fmaf(w[0], xv, acc[0][t]);
                acc[1][t] = fmaf(w[1], xv, acc[1][t]);
            }
        }
    } else {
        const uint32_t nchunk = (uint32_t)(args.ne0 / 32);
        for (uint32_t c = lane; c < nchunk; c += 64) {
            float w[2][32];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                if (r < nr) decode_chunk<FMT>(M.W + (uint64_t)(r0 + r) * rb, c, w[r]);
                else {
#pragma unroll
                    for (int j = 0; j < 32; j++) w[r][j] = 0.0f;
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (t >= args.ntok) break;
                const float4 *xp = (const float4 *)(args.x + (uint64_t)t * args.ldx + (uint64_t)c * 32);
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float4 v = xp[j];
                    s0 = fmaf(w[0][4 * j], v.x, s0); s0 = fmaf(w[0][4 * j + 1], v.y, s0);
                    s0 = fmaf(w[0][4 * j + 2], v.z, s0); s0 = fmaf(w[0][4 * j + 3], v.w, s0);
                    s1 = fmaf(w[1][4 * j], v.x, s1); s1 = fmaf(w[1][4 * j + 1], v.y, s1);
                    s1 = fmaf(w[1][4 * j + 2], v.z, s1); s1 = fmaf(w[1][4 * j + 3], v.w, s1);
                }
                acc[0][t] += s0;
                acc[1][t] += s1;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float v = acc[r][t];
#pragma unroll
            for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
            acc[r][t] = v;
        }
    if (lane == 0)
        for (int r = 0; r < nr; r++) {
            const uint32_t row = r0 + r;
            if (row < M.row_lo) continue;
            for (int t = 0; t < NT && t < args.ntok; t++) {
                float *o = M.out + (uint64_t)t * M.ldo + row;
                const float v = args.rss ? acc[r][t] * rsc[t] : acc[r][t];
                *o = (args.flags & QGPU_GEMV_ACCUM) ? *o + v : v;
            }
        }
}

// ---------------------------------------------------------------- launchers
// Validates an activation transform for n rows of ne0 and launches its prep
// kernel: digit planes into the workspace when `digits`, fp32 rows into xout.
// defer: single-segment RMSNORM is prepared as x*w plus per-super-block sums of
// squares (ws_rss) for the GEMV to apply the row factor; *deferred = 1 tells the caller.
// defer2: the two-segment RMSNORM without xout likewise, [x*w | y*w2] with one factor per
// half (*deferred = 2; for matrix-core GEMVs with no K split only: the caller says).
static int prep_act(const GemvExec &ex, const qgpu_act *act, int n, uint64_t ne0, int digits, bool defer = false,
                    int *deferred = nullptr, bool defer2 = false)
{
    if (deferred) *deferred = 0;
    if (!act || (!act->x && !act->embd) || n < 1 || n > QGPU_MAX_B) return QGPU_E_ARG;
    if (ne0 % 256 || (digits && ne0 > MAX_K)) return QGPU_E_RANGE;
    ActDev d = {};
    d.x = act->x; d.y = act->y; d.w = act->w; d.w2 = act->w2; d.xout = act->xout;
    d.ldx = act->ldx; d.ldy = act->ldy; d.ldxo = act->ldxo; d.eps = act->eps; d.ntok = n; d.digits = digits;
    const bool rows = n > 1;
    const bool single = act->kind == QGPU_ACT_RMSNORM && (!act->seg || act->seg == ne0);
    const bool gath = act->embd != nullptr;
    if (gath) {                          // x gathered from embedding rows (RMSNORM, the first segment)
        const qgpu_tensor *Em = act->embd;
        if (act->kind != QGPU_ACT_RMSNORM || !act->tok || Em->type != T_IQ4_XS || !Em->packed || act->n_part ||
            Em->ne0 != (single ? ne0 : act->seg))
            return QGPU_E_ARG;
        d.embd = (const uint8_t *)Em->data; d.tok = act->tok; d.embd_ne1 = Em->ne1;
    }
    if (act->n_part < 0 || act->n_part > 8) return QGPU_E_ARG;
    if ((act->n_part || act->xnew) && !(single && defer)) return QGPU_E_ARG;   // deferred RMSNORM only
    if (act->n_part && (!act->part || (rows && act->ldp < ne0))) return QGPU_E_ARG;
    if (act->xnew && rows && act->ldxn < ne0) return QGPU_E_ARG;
    if (single && defer) {
        if (!act->w || (!gath && rows && act->ldx < ne0) || (act->xout && rows && act->ldxo < ne0)) return QGPU_E_ARG;
        d.part = act->part; d.ldp = act->ldp; d.pstride = (uint64_t)n * act->ldp; d.n_part = act->n_part;
        d.xnew = act->xnew; d.ldxn = act->ldxn; d.rss = ws_rss(ex); d.nsb = (int)(ne0 / 256);
        const dim3 grid((unsigned)(ne0 / 256), (unsigned)n);
        uint8_t *A = ex.ws;
        float *xs = (float *)(ex.ws + 2 * PLANE_BYTES);
#define PT_NP(NP_) case NP_: hipLaunchKernelGGL((k_prep_tok<ACT_RMS_DEFER, NP_>), grid, dim3(256), 0, ex.st, d, A, xs); break
        if (gath) hipLaunchKernelGGL((k_prep_tok<ACT_RMS_EMBD, 0>), grid, dim3(256), 0, ex.st, d, A, xs);
        else switch (act->n_part) {
        PT_NP(0); PT_NP(1); PT_NP(2); PT_NP(3); PT_NP(4); PT_NP(5); PT_NP(6); PT_NP(7); default: PT_NP(8);
        }
#undef PT_NP
        QG_LAUNCH_CHECK();
        if (deferred) *deferred = 1;
        return QGPU_OK;
    }
    if (defer2 && digits && act->kind == QGPU_ACT_RMSNORM && act->seg && 2 * act->seg == ne0 && !act->xout &&
        act->seg % 256 == 0) {
        if (!act->w || !act->w2 || !act->y || (rows && act->ldy < act->seg) || (!gath && rows && act->ldx < act->seg))
            return QGPU_E_ARG;
        d.seg = act->seg; d.rss = ws_rss(ex); d.nsb = (int)(ne0 / 256);
        hipLaunchKernelGGL((k_prep_tok<ACT_RMS_CAT, 0>), dim3((unsigned)(ne0 / 256), (unsigned)n), dim3(256), 0, ex.st,
                           d, ex.ws, (float *)(ex.ws + 2 * PLANE_BYTES));
        QG_LAUNCH_CHECK();
        if (deferred) *deferred = 2;
        return QGPU_OK;
    }
    if (act->xout && rows && act->ldxo < ne0) return QGPU_E_ARG;
    uint64_t wx = ne0;                                    // columns read from x
    switch (act->kind) {
    case QGPU_ACT_COPY: break;
    case QGPU_ACT_RMSNORM: {
        d.seg = act->seg ? act->seg : ne0;
        if ((d.seg != ne0 && 2 * d.seg != ne0) || d.seg % 256 || !act->w) return QGPU_E_ARG;
        if (d.seg != ne0 && (!act->y || !act->w2 || (rows && act->ldy < d.seg) || act->ldy % 4 ||
                             ((uintptr_t)act->y & 15)))
            return QGPU_E_ARG;
        if (!gath && (act->ldx % 4 || ((uintptr_t)act->x & 15))) return QGPU_E_ARG;   // float4 row sums
        wx = d.seg;
        break;
    }
    case QGPU_ACT_SILU_MUL:
        if (!act->y || (rows && act->ldy < ne0)) return QGPU_E_ARG;
        break;
    case QGPU_ACT_GATED_NORM:
        d.seg = act->seg;
        if (!act->y || !act->w || (rows && act->ldy < ne0) || (d.seg != 64 && d.seg != 128 && d.seg != 256))
            return QGPU_E_ARG;
        break;
    default: return QGPU_E_ARG;
    }
    if (!gath && rows && act->ldx < wx) return QGPU_E_ARG;
    const dim3 grid((unsigned)(ne0 / 256), (unsigned)n);                  // one token per block
    uint8_t *A = ex.ws;
    float *xs = (float *)(ex.ws + 2 * PLANE_BYTES);
    switch (act->kind) {
    case QGPU_ACT_COPY: hipLaunchKernelGGL((k_prep_tok<QGPU_ACT_COPY, 0>), grid, dim3(256), 0, ex.st, d, A, xs); break;
    case QGPU_ACT_RMSNORM:                                                     // four tokens per block
        if (gath)
            hipLaunchKernelGGL(k_prep_rms<true>, dim3((unsigned)(ne0 / 256), (unsigned)(n > 4 ? 2 : 1)), dim3(256), 0, ex.st, d, A, xs);
        else
            hipLaunchKernelGGL(k_prep_rms<false>, dim3((unsigned)(ne0 / 256), (unsigned)(n > 4 ? 2 : 1)), dim3(256), 0, ex.st, d, A, xs);
        break;
    case QGPU_ACT_SILU_MUL: hipLaunchKernelGGL((k_prep_tok<QGPU_ACT_SILU_MUL, 0>), grid, dim3(256), 0, ex.st, d, A, xs); break;
    default: hipLaunchKernelGGL((k_prep_tok<QGPU_ACT_GATED_NORM, 0>), grid, dim3(256), 0, ex.st, d, A, xs); break;
    }
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

// One launch for the matrices idx[0..cnt) of one format.  IQ4_XS reads the
// digit planes already in the workspace; the other formats read fp32 rows x.
// one matrix-core GEMV launch: format FMT, NA digit planes, nw waves per tile, MODE bits
template <int FMT>
static void launch_mfma(const GemvExec &ex, const GemvArgs &A, uint32_t blocks, int na, int nw, int mode)
{
#define MF_GO(NA_, NW_, M_) hipLaunchKernelGGL((k_gemv_mfma<FMT, NA_, NW_, M_>), dim3(blocks), dim3(64 * NW_), 0, ex.st, A)
#define MF_NW(NA_, M_) do { if (nw == 1) MF_GO(NA_, 1, M_); else if (nw == 2) MF_GO(NA_, 2, M_); \
                            else if (nw == 3) MF_GO(NA_, 3, M_); else if (nw == 4) MF_GO(NA_, 4, M_); \
                            else MF_GO(NA_, 8, M_); } while (0)
#define MF_MODE(NA_) do { if (mode == 0) MF_NW(NA_, 0); else if (mode == IQ4_RMS) MF_NW(NA_, IQ4_RMS); \
                          else if (mode == IQ4_SPLIT) MF_NW(NA_, IQ4_SPLIT); \
                          else if (mode == IQ4_PAIR) MF_NW(NA_, IQ4_PAIR); \
                          else if (mode == (IQ4_RMS | IQ4_PAIR)) MF_NW(NA_, IQ4_RMS | IQ4_PAIR); \
                          else if (mode == IQ4_RMS2) MF_NW(NA_, IQ4_RMS2); \
                          else if (mode == (IQ4_RMS2 | IQ4_PAIR)) MF_NW(NA_, IQ4_RMS2 | IQ4_PAIR); \
                          else MF_NW(NA_, IQ4_RMS | IQ4_SPLIT); } while (0)
    // the ring-less instances exist for IQ4_XS, one plane, 3, 4 or 8 waves per tile, K-split or
    // pair-split launches (launch_group asks for no other); anything else runs its ring instance
    const int m = mode & ~IQ4_NORING;
    const bool nr = (mode & IQ4_NORING) && FMT == T_IQ4_XS && na == 1 && (nw == 3 || nw == 4 || nw == 8) &&
                    (m == IQ4_SPLIT || m == IQ4_PAIR || m == (IQ4_RMS | IQ4_PAIR) || m == (IQ4_RMS | IQ4_SPLIT));
    if (nr) {
        if constexpr (FMT == T_IQ4_XS) {
#define MF_NR(M_) do { if (nw == 3) MF_GO(1, 3, M_ | IQ4_NORING); else if (nw == 8) MF_GO(1, 8, M_ | IQ4_NORING); \
                       else MF_GO(1, 4, M_ | IQ4_NORING); } while (0)
            if (m == IQ4_SPLIT) MF_NR(IQ4_SPLIT);
            else if (m == IQ4_PAIR) MF_NR(IQ4_PAIR);
            else if (m == (IQ4_RMS | IQ4_PAIR)) MF_NR(IQ4_RMS | IQ4_PAIR);
            else MF_NR(IQ4_RMS | IQ4_SPLIT);
#undef MF_NR
        }
    } else {
        mode = m;
        if (na == 1) MF_MODE(1); else MF_MODE(2);
    }
#undef MF_MODE
#undef MF_NW
#undef MF_GO
}

template <int FMT>
static void launch_wide(const GemvExec &ex, const GemvArgs &A, uint32_t blocks, int na, int mode)
{
#define WG_GO(NA_, M_) hipLaunchKernelGGL((k_gemv_wide<FMT, NA_, M_>), dim3(blocks), dim3(64 * WIDE_NW(FMT, NA_)), 0, \
                                          ex.st, A)
    if (na == 1) { if (mode) WG_GO(1, IQ4_RMS); else WG_GO(1, 0); }
    else { if (mode) WG_GO(2, IQ4_RMS); else WG_GO(2, 0); }
#undef WG_GO
}

// Blocks of one kernel instance that a compute unit holds at once (its VGPRs set the waves
// per SIMD), from the runtime's occupancy calculator; cached per instance.
template <int FMT, int NA, int NW, int M>
static int mfma_resident()
{
    static int nb = -1;
    if (nb < 0) {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, (const void *)k_gemv_mfma<FMT, NA, NW, M>, 64 * NW, 0) !=
            hipSuccess)
            v = 0;
        nb = v;
    }
    return nb;
}
template <int FMT>
static int mfma_resident_of(int na, int nw, int mode)
{
#define MR_NW(NA_, M_) (nw == 2 ? mfma_resident<FMT, NA_, 2, M_>() : nw == 3 ? mfma_resident<FMT, NA_, 3, M_>() \
                                  : mfma_resident<FMT, NA_, 4, M_>())
#define MR_MODE(NA_) (mode == 0 ? MR_NW(NA_, 0) : mode == IQ4_RMS ? MR_NW(NA_, IQ4_RMS) \
                      : mode == IQ4_SPLIT ? MR_NW(NA_, IQ4_SPLIT) : mode == IQ4_PAIR ? MR_NW(NA_, IQ4_PAIR) \
                      : mode == (IQ4_RMS | IQ4_PAIR) ? MR_NW(NA_, IQ4_RMS | IQ4_PAIR) \
                      : mode == IQ4_RMS2 ? MR_NW(NA_, IQ4_RMS2) : mode == (IQ4_RMS2 | IQ4_PAIR) ? MR_NW(NA_, IQ4_RMS2 | IQ4_PAIR) \
                      : MR_NW(NA_, IQ4_RMS | IQ4_SPLIT))
    return na == 1 ? MR_MODE(1) : MR_MODE(2);
#undef MR_MODE
#undef MR_NW
}
static int mfma_resident_fmt(int type, int na, int nw, int mode)
{
    switch (type) {
    case T_IQ4_XS: return mfma_resident_of<T_IQ4_XS>(na, nw, mode);
    case T_Q4_K: return mfma_resident_of<T_Q4_K>(na, nw, mode);
    case T_Q5_K: return mfma_resident_of<T_Q5_K>(na, nw, mode);
    case T_Q6_K: return mfma_resident_of<T_Q6_K>(na, nw, mode);
    case T_Q8_0: return mfma_resident_of<T_Q8_0>(na, nw, mode);
    default: return 0;
    }
}

#ifndef NW8_TILES
#define NW8_TILES 512       // grids of at most this many tiles (no K split) run 8 waves per tile; with 1100
                            // or 1280 the plain 17408x5120 B=4 GEMV alone is 3% faster, but the 27B step
                            // (896..1088-tile GEMVs with row factors) 1.6% slower
#endif
static int launch_group(const GemvExec &ex, const qgpu_tensor *const *Ws, const int *idx, int cnt, const float *x,
                        uint64_t ldx, int n, float *const *outs, const uint64_t *ldos, int flags, const uint64_t *r0s,
                        const uint64_t *r1s, int ks, const int *ksm, float eps, int deferred)
{
    const qgpu_tensor *W0 = Ws[idx[0]];
    GemvArgs A = {};
    A.n_mat = cnt; A.ntok = n; A.flags = flags; A.x = x; A.ldx = ldx; A.ne0 = W0->ne0;
    if (deferred) {          // 1: one row factor; 2: one per half of the row (the two-segment RMSNORM)
        A.rss = ws_rss(ex); A.rss_nsb = (int)(W0->ne0 / 256); A.eps = eps;
        A.rss_seg = deferred == 2 ? A.rss_nsb / 2 : 0;
        A.rss_inv_n = 1.0f / (float)(deferred == 2 ? W0->ne0 / 2 : W0->ne0);
    }
    A.nsb = (int)(W0->ne0 / 256);
    const bool mfma = W0->packed;
    const uint32_t per = mfma ? IQ4_TILE_ROWS : 8;
    uint32_t tiles = 0, blocks = 0;
    bool split = false;
    for (int j = 0; j < cnt; j++) {
        const qgpu_tensor *W = Ws[idx[j]];
        const uint64_t lo = r0s ? r0s[idx[j]] : 0, hi = r1s ? r1s[idx[j]] : W->ne1;
        const uint32_t t = (uint32_t)((hi + per - 1) / per - lo / per);
        const int kj = ksm ? ksm[idx[j]] : ks;                 // K ranges per tile of this matrix
        GemvMat &M = A.m[j];
        M.W = (const uint8_t *)W->data;
        M.out = outs[idx[j]];
        M.ldo = ldos[idx[j]];
        M.rows = (uint32_t)W->ne1;
        M.row_lo = (uint32_t)lo;
        M.row_hi = (uint32_t)hi;
        M.tile_first = (uint32_t)(lo / per);
        M.tile0 = tiles;
        M.blk0 = blocks;
        M.ks = (uint32_t)kj;
        M.pstride = (uint64_t)n * ldos[idx[j]];
        tiles += t;
        blocks += t * (uint32_t)kj;
        if (kj > 1) split = true;
    }
    if (!tiles) return QGPU_OK;
    A.pair0 = tiles;
    if (mfma) {
        if (W0->ne0 > MAX_K) return QGPU_E_RANGE;
#ifndef GEMV_WIDE
#define GEMV_WIDE 1
#endif
#ifndef WIDE_MIN_TILES
#define WIDE_MIN_TILES 4096   // tiles from which one matrix with its activations in LDS takes k_gemv_wide
#endif
        // one wide matrix, no K split, its digit planes within the LDS operand: k_gemv_wide, all its
        // blocks resident at once (pair0 = the launch's tile count).  It pays where the per-tile
        // kernel re-reads whole digit planes, B = 4 and 8; 248,320 x 5120 through gemv_batch (us,
        // per-tile -> wide): IQ4_XS B = 4 143.7 -> 133.7, B = 8 192.6 -> 187.3; Q4_K 144.6 -> 138.1,
        // 195.7 -> 188.8; Q5_K B = 8 223.4 -> 220.0; Q8_0 B = 8 275.2 -> 249.6.  Not taken: B = 1, 2
        // (IQ4_XS 133.0 -> 139.4), B = 5, 6 (IQ4_XS 177.4 -> 191.0, plane 2 partly empty), Q5_K at B = 4
        // (+0.5%), Q8_0 below 7 tokens, Q6_K (too few waves for its VGPRs).
        {
            const int na = n > 4 ? 2 : 1, t = W0->type;
            const bool fmt_ok = n == 4 ? (t == T_IQ4_XS || t == T_Q4_K)
                                       : n == 8 && (t == T_IQ4_XS || t == T_Q4_K || t == T_Q5_K || t == T_Q8_0);
            if (GEMV_WIDE && fmt_ok && cnt == 1 && !split && ks == 1 && !A.rss_seg && tiles >= WIDE_MIN_TILES && ex.n_cu > 0 &&
                A.nsb <= (na == 1 ? WIDE_NSB(1) : WIDE_NSB(2))) {
                A.A = ex.ws;
                A.xs = (const float *)(ex.ws + 2 * PLANE_BYTES);
                const int mode = A.rss ? IQ4_RMS : 0;
                const uint32_t blocks = (uint32_t)ex.n_cu * WIDE_BPC(na);
                switch (W0->type) {
                case T_IQ4_XS: launch_wide<T_IQ4_XS>(ex, A, blocks, na, mode); break;
                case T_Q4_K: launch_wide<T_Q4_K>(ex, A, blocks, na, mode); break;
                case T_Q5_K: launch_wide<T_Q5_K>(ex, A, blocks, na, mode); break;
                case T_Q6_K: launch_wide<T_Q6_K>(ex, A, blocks, na, mode); break;
                case T_Q8_0: launch_wide<T_Q8_0>(ex, A, blocks, na, mode); break;
                default: return QGPU_E_TYPE;
                }
                QG_LAUNCH_CHECK();
                return QGPU_OK;
            }
        }
#ifndef GEMV_PAIR_SPLIT
#define GEMV_PAIR_SPLIT 1
#endif
        // Tail balance: with every block resident, a launch ends when the compute units holding
        // one tile more than the others finish.  When the tiles are r > 0 over a multiple of the
        // compute units (r at most half of them), the last r tiles run as two half-K blocks each,
        // so those units stream half a tile more instead of a whole one (17408 x 5120: 1024 + 64
        // tiles).  Not with a K split of the caller's (partial planes) or per-matrix splits.
        const uint32_t ncu = ex.n_cu > 0 ? (uint32_t)ex.n_cu : 0;
        if (GEMV_PAIR_SPLIT && ncu && !split && ks == 1 && A.nsb >= 2 && tiles > ncu) {
            const uint32_t r = tiles % ncu;
            if (r && r <= ncu / 2 && r <= PAIR_MAX_TILES) {
                A.pair0 = tiles - r;
                A.xchg = ws_xchg(ex);
                blocks = tiles + r;
            }
        }
        const int na = n > 4 ? 2 : 1;
        A.A = ex.ws;
        A.xs = (const float *)(ex.ws + 2 * PLANE_BYTES);
        // waves per tile (K split inside the block).  Measured on MI355X over the
        // model's shapes with the 3/1 prefetch rings: 4 waves is best or within
        // noise everywhere except narrow outputs (<= 512 tiles, e.g. 5120 rows,
        // fewer blocks than 2 per CU), where 8 waves per tile hide more latency.
        // QGPU_GEMV_NW=1|2|3|4|8 forces the split.
        static int force_nw = -1;
        if (force_nw < 0) {
            const char *e = getenv("QGPU_GEMV_NW");
            force_nw = e ? atoi(e) : 0;
        }
#ifndef GEMV_NORING_MIN_B
#define GEMV_NORING_MIN_B 3
#endif
#ifndef GEMV_NORING_MAX_TPC
#define GEMV_NORING_MAX_TPC 12
#endif
#ifndef NW8_TILES_NA2
#define NW8_TILES_NA2 1100  // two-plane launches of at most this many tiles run 8 waves per tile
#endif
#ifndef NW8_TILES_NR
#define NW8_TILES_NR 2200   // ring-less launches of at most this many tiles run 8 waves per tile
#endif
        // Prefetch rings off for the verify-sized launches of IQ4_XS with one digit plane and 3 or 4
        // tokens (up to 12 tiles per compute unit: not the lm_head).  Same-box A/B of the 27B model:
        // verify B = 4 5.19 / 5.21 -> 5.15 / 5.16 ms, spec decode 171.0 / 170.6 -> 171.8 / 171.4 tok/s,
        // the 17408 x 5120 GEMV 13.45 -> 13.35-13.39 us; at B = 1 (decode 4.67 -> 4.69 ms, MTP draft
        // 0.211 -> 0.215 ms) and with two digit planes (verify B = 6 and 8 +0.2-0.3%) the rings pay.
        // (Rings whose waits let the next step's loads stay in flight through a step -- dead loads
        // past the last step, so that every path issues the same loads -- measured slower still:
        // 15.1-15.2 us for that GEMV.)
        // Only the K-split and pair-split instances (the model's verify launches and the 17408 x 5120
        // GEMV): without the rings the plain and row-factor ones take 98-102 VGPRs, 4 waves per SIMD.
        // A K split over more than 32 super-blocks (ffn_down, K = 17408: 17 per block) keeps them:
        // spec decode 171.6-171.7 -> 172.0-172.1 tok/s (same box).
        const bool noring = W0->type == T_IQ4_XS && na == 1 && n >= GEMV_NORING_MIN_B && (split || A.pair0 < tiles) &&
                            !A.rss_seg && !(split && A.nsb > 32) && ex.n_cu > 0 &&
                            tiles <= (uint32_t)GEMV_NORING_MAX_TPC * (uint32_t)ex.n_cu;
        // 8 waves per tile for the ring-less launches (attention q/k/v 896 tiles, GDN input 1030, the
        // 17408 x 5120 GEMV 1088: verify B = 4 5.14-5.16 -> 5.12-5.13 ms; FFN gate+up 2176 as well:
        // 5.115-5.120 -> 5.110-5.112 ms, same box); at B = 1 the ring kernels of these grids stay at 4
        // (decode 4.65 -> 4.69 ms with 8)
        // Two digit planes (5-8 tokens) take 8 waves per tile up to 1100 tiles with a row factor (the
        // model's attention q/k/v and GDN input: 8192 positions, verify k = 7 6.69 -> 6.62-6.65 ms, same
        // box; the 2176-tile FFN gate+up keeps 4, with 8 k = 5 6.31-6.33 -> 6.36-6.38 ms) and for the
        // K-quants (gemv_batch B = 8, 17408 x 5120: Q4_K / Q5_K / Q6_K +6-10%; IQ4_XS and Q8_0 without
        // a row factor -3% / -5%, so those keep 4).
        const bool na2w8 = na == 2 && (A.rss || W0->type == T_Q4_K || W0->type == T_Q5_K || W0->type == T_Q6_K);
        int nw = (ks == 1 && tiles <= (noring ? NW8_TILES_NR : na2w8 ? NW8_TILES_NA2 : NW8_TILES)) ? 8 : 4;
        if (force_nw >= 1 && force_nw <= 4) nw = force_nw;
        if (force_nw == 8) nw = 8;
        while (nw > 1 && A.nsb / ks < nw) nw >>= 1;         // no idle waves on short K ranges
        if (A.rss && nw < 3) nw = 4;                        // row factors: <= 3 tokens per wave
        int mode = (A.rss ? (A.rss_seg ? IQ4_RMS2 : IQ4_RMS) : 0) | (split ? IQ4_SPLIT : 0) |
                         (A.pair0 < tiles ? IQ4_PAIR : 0);
#ifndef GEMV_NW3_RESIDENT
#define GEMV_NW3_RESIDENT 1
#endif
#ifndef GEMV_NW_MIN_RESIDENT
#define GEMV_NW_MIN_RESIDENT 3   // 2 waves per tile measured slower than a second round of blocks
#endif
        // Residency: when the compute units cannot hold every 4-wave block at once (the kernel's
        // VGPRs cap the waves per SIMD), the blocks left over start only as the first ones end,
        // a second round at the end of the launch; 3 waves per tile (longer K slices) then fit
        // them all where they can (the GDN input projection at B = 5..8 with 4 waves per tile:
        // 1144 blocks against 4 x 256 resident 4-wave blocks, 5 x 256 3-wave blocks; it now
        // takes 8, above).
        if (GEMV_NW3_RESIDENT && nw == 4 && force_nw == 0 && ex.n_cu > 0 &&
            (long)blocks > (long)mfma_resident_fmt(W0->type, na, 4, mode) * ex.n_cu) {
            for (int w = 3; w >= GEMV_NW_MIN_RESIDENT; w--)
                if (A.nsb / ks >= w && (long)blocks <= (long)mfma_resident_fmt(W0->type, na, w, mode) * ex.n_cu) {
                    nw = w;
                    break;
                }
        }
        if (noring && (nw == 3 || nw == 4 || nw == 8)) mode |= IQ4_NORING;
        switch (W0->type) {
        case T_IQ4_XS: launch_mfma<T_IQ4_XS>(ex, A, blocks, na, nw, mode); break;
        case T_Q4_K: launch_mfma<T_Q4_K>(ex, A, blocks, na, nw, mode); break;
        case T_Q5_K: launch_mfma<T_Q5_K>(ex, A, blocks, na, nw, mode); break;
        case T_Q6_K: launch_mfma<T_Q6_K>(ex, A, blocks, na, nw, mode); break;
        case T_Q8_0: launch_mfma<T_Q8_0>(ex, A, blocks, na, nw, mode); break;
        default: return QGPU_E_TYPE;
        }
        QG_LAUNCH_CHECK();
        return QGPU_OK;
    }
#define VALU_CASE(F)                                                                                              \
    case F:                                                                                                       \
        switch (n) {                                                                                              \
        case 1: hipLaunchKernelGGL((k_gemv_valu<F, 1>), dim3(tiles), dim3(256), 0, ex.st, A); break;        \
        case 2: hipLaunchKernelGGL((k_gemv_valu<F, 2>), dim3(tiles), dim3(256), 0, ex.st, A); break;        \
        case 3: case 4: hipLaunchKernelGGL((k_gemv_valu<F, 4>), dim3(tiles), dim3(256), 0, ex.st, A); break; \
        default: hipLaunchKernelGGL((k_gemv_valu<F, 8>), dim3(tiles), dim3(256), 0, ex.st, A); break;      \
        }                                                                                                         \
        break;
    switch (W0->type) {
        VALU_CASE(T_F32)
        VALU_CASE(T_Q8_0)
        VALU_CASE(T_Q4_K)
        VALU_CASE(T_Q5_K)
        VALU_CASE(T_Q6_K)
    default: return QGPU_E_TYPE;
    }
#undef VALU_CASE
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

// act == NULL: packed matrices only, on the digit planes of the last prepare.
static int gemv_multi_on(const GemvExec &ex, const qgpu_tensor *const *Ws, int n_mat, const qgpu_act *act, int n,
                         float *const *outs, const uint64_t *ldos, int flags, const uint64_t *r0s,
                         const uint64_t *r1s, int ks = 1, const int *ksm = nullptr)
{
    int rc = QGPU_OK;
    if (!Ws || !outs || !ldos || n_mat < 1 || n_mat > QGPU_MAX_MULTI || n < 1 || n > QGPU_MAX_B || !Ws[0])
        return QGPU_E_ARG;
    const uint64_t ne0 = Ws[0]->ne0;
    bool any_mfma = false, any_valu = false;
    for (int j = 0; j < n_mat; j++) {
        if (!Ws[j] || !outs[j] || Ws[j]->ne0 != ne0) return QGPU_E_ARG;
        if (n > 1 && ldos[j] < (r1s ? r1s[j] : Ws[j]->ne1)) return QGPU_E_ARG;
        if (r0s && (r0s[j] > r1s[j] || r1s[j] > Ws[j]->ne1)) return QGPU_E_ARG;
        if (Ws[j]->packed) any_mfma = true; else any_valu = true;
    }
    if (ks < 1 || ks > 8 || (ks > 1 && (n_mat != 1 || any_valu || r0s || (int)(ne0 / 256) < ks))) return QGPU_E_ARG;
    if (ksm) {                                              // per-matrix K split (packed formats, plain outputs)
        if (ks != 1 || (flags & QGPU_GEMV_ACCUM)) return QGPU_E_ARG;
        for (int j = 0; j < n_mat; j++)
            if (ksm[j] < 1 || ksm[j] > QGPU_MAX_KS || (int)(ne0 / 256) < ksm[j] || (ksm[j] > 1 && !Ws[j]->packed))
                return QGPU_E_ARG;
    }
    const float *xv = nullptr;                              // fp32 rows for the VALU kernel (unpacked formats)
    uint64_t ldxv = ne0;
    int deferred = 0;
    if (!act) {
        if (any_valu) return QGPU_E_TYPE;
    } else {
        const bool xform = act->kind != QGPU_ACT_COPY;
        if (any_valu) {
            xv = xform ? act->xout : act->x;
            ldxv = xform ? act->ldxo : act->ldx;
            if (!xv || (n > 1 && ldxv < ne0)) return QGPU_E_ARG;
            if (ldxv % 4 || ((uintptr_t)xv & 15)) return QGPU_E_ARG;   // float4 activation loads
        }
        if (any_mfma || xform) {
            if (!any_mfma && ne0 % 256) return QGPU_E_RANGE;
            // row factors: <= 64 sums; two per row only for matrix-core GEMVs with no K split
            rc = prep_act(ex, act, n, ne0, any_mfma ? 1 : 0, ne0 <= 64 * 256, &deferred,
                          ne0 <= 64 * 256 && !any_valu && ks == 1 && !ksm);
            if (rc) return rc;
        }
    }
    const float eps = act ? act->eps : 0.0f;
    // group matrices of the same format (one launch per group)
    int done[QGPU_MAX_MULTI] = {0};
    for (int j = 0; j < n_mat; j++) {
        if (done[j]) continue;
        int idx[QGPU_MAX_MULTI], cnt = 0;
        for (int i = j; i < n_mat; i++)
            if (!done[i] && Ws[i]->type == Ws[j]->type) { idx[cnt++] = i; done[i] = 1; }
        rc = launch_group(ex, Ws, idx, cnt, xv, ldxv, n, outs, ldos, flags, r0s, r1s, ks, ksm, eps, deferred);
        if (rc) return rc;
    }
    return QGPU_OK;
}

// the library entry points: library stream and workspace
static int gemv_multi(const qgpu_tensor *const *Ws, int n_mat, const qgpu_act *act, int n, float *const *outs,
                      const uint64_t *ldos, int flags, const uint64_t *r0s, const uint64_t *r1s, int ks = 1)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    return gemv_multi_on(lib_exec(), Ws, n_mat, act, n, outs, ldos, flags, r0s, r1s, ks);
}

static qgpu_act copy_act(const float *x, uint64_t ldx)
{
    qgpu_act a = {};
    a.kind = QGPU_ACT_COPY;
    a.x = x;
    a.ldx = ldx;
    return a;
}

extern "C" int qgpu_gemv_batch(const qgpu_tensor *W, const float *x, uint64_t ldx, int n, float *out,
                               uint64_t ldo, int flags)
{
    if (!x || !W || (n > 1 && ldx < W->ne0)) return QGPU_E_ARG;
    const qgpu_act a = copy_act(x, ldx);
    return gemv_multi(&W, 1, &a, n, &out, &ldo, flags, nullptr, nullptr);
}

// ---------------------------------------------------------------- allocation-free gemv_batch
// For callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc): the workspace of the
// batched GEMV (two 4-token digit planes for up to MAX_K = 65536 columns, their
// conversion factors, the deferred-RMSNorm sums and the exchange slots of the
// pair-split tiles: 1,875,968 bytes) lives in this file-scope device array, one
// copy per GPU, held until the process ends.  Its device address is looked up
// once per device with hipGetSymbolAddress; the host-side name is never passed
// to a kernel.  Every call on a GPU shares that GPU's copy, so calls that
// overlap on one GPU (two streams, two threads) race.  Each call writes the
// digit tiles and factors of every super-block it reads before the GEMV reads
// them; the exchange slots start at zero (static storage) and every launch
// leaves them at zero.
static __device__ __align__(256) uint8_t scratch[GEMV_WS_BYTES];
#define SCRATCH_MAX_DEV 64
static uint8_t *scratch_ptr[SCRATCH_MAX_DEV];
static int scratch_ncu[SCRATCH_MAX_DEV];

extern "C" int qgpu_gemv_batch_noalloc(const qgpu_tensor *W, const float *x, uint64_t ldx, int n, float *out,
                                       uint64_t ldo, int flags, void *stream)
{
    if (!x || !W || !out || n < 1 || n > QGPU_MAX_B || (n > 1 && (ldx < W->ne0 || ldo < W->ne1)))
        return QGPU_E_ARG;
    if (W->ne0 > MAX_K) return QGPU_E_RANGE;              // the digit planes hold MAX_K columns
    int dev = -1;
    QG_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= SCRATCH_MAX_DEV) return QGPU_E_RANGE;
    if (!scratch_ptr[dev]) {                              // first call on this device: its copy's address
        void *p = nullptr;
        int ncu = 0;
        QG_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        QG_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
        if (!p) return QGPU_E_INIT;
        scratch_ncu[dev] = ncu;
        scratch_ptr[dev] = (uint8_t *)p;
    }
    const GemvExec ex{ (hipStream_t)stream, scratch_ptr[dev], scratch_ncu[dev] };
    const qgpu_act a = copy_act(x, ldx);
    return gemv_multi_on(ex, &W, 1, &a, n, &out, &ldo, flags, nullptr, nullptr);
}

extern "C" int qgpu_gemv_multi_batch(const qgpu_tensor *const *Ws, int n_mat, const float *x, uint64_t ldx, int n,
                                     float *const *outs, const uint64_t *ldos, int flags)
{
    if (!x || !Ws || !Ws[0] || (n > 1 && ldx < Ws[0]->ne0)) return QGPU_E_ARG;
    const qgpu_act a = copy_act(x, ldx);
    return gemv_multi(Ws, n_mat, &a, n, outs, ldos, flags, nullptr, nullptr);
}

extern "C" int qgpu_gemv_act_batch(const qgpu_tensor *const *Ws, int n_mat, const qgpu_act *act, int n,
                                   float *const *outs, const uint64_t *ldos, int flags)
{
    if (!act) return QGPU_E_ARG;
    return gemv_multi(Ws, n_mat, act, n, outs, ldos, flags, nullptr, nullptr);
}

extern "C" int qgpu_gemv_act_batch_ks(const qgpu_tensor *const *Ws, int n_mat, const qgpu_act *act, int n,
                                      float *const *outs, const uint64_t *ldos, const int *ks)
{
    if (!act || !ks) return QGPU_E_ARG;
    int rc = qg::ensure_init();
    if (rc) return rc;
    return gemv_multi_on(lib_exec(), Ws, n_mat, act, n, outs, ldos, 0, nullptr, nullptr, 1, ks);
}

extern "C" int qgpu_gemv_act_split(const qgpu_tensor *W, const qgpu_act *act, int n, float *part, uint64_t ldp,
                                   int ks)
{
    if (!act || !W || !part || !W->packed) return QGPU_E_ARG;
    if (n > 1 && ldp < W->ne1) return QGPU_E_ARG;
    if (ks == 1) return gemv_multi(&W, 1, act, n, &part, &ldp, 0, nullptr, nullptr, 1);
    return gemv_multi(&W, 1, act, n, &part, &ldp, 0, nullptr, nullptr, ks);
}

// Splits narrow IQ4_XS matrices so that the blocks (tiles x ks, 4 waves each)
// cover the compute units about 4-5 times; measured on MI355X: 5120 x 17408
// runs best at ks 4, 5120 x 6144 at ks 2..4 (a single-pass grid of 320 tiles
// leaves 1.6x more work on the CUs that get two tiles).
#ifndef SPLIT_TARGET
#define SPLIT_TARGET 1280   // blocks a K-split GEMV of a narrow output aims at (5 per CU); measured over the
                            // 27B step: 640 (ks 2) 2% and 2560 (ks 8) 1% slower
#endif
extern "C" int qgpu_gemv_split_ks(const qgpu_tensor *W)
{
    if (!W || !W->packed) return 1;
    const uint64_t tiles = (W->ne1 + IQ4_TILE_ROWS - 1) / IQ4_TILE_ROWS, nsb = W->ne0 / 256;
    if (tiles > 640) return 1;
    int ks = (int)(SPLIT_TARGET / tiles);
    if (ks > 8) ks = 8;
    while (ks > 1 && (uint64_t)ks * 4 > nsb) ks--;          // at least 4 super-blocks per block
    return ks < 1 ? 1 : ks;
}

__global__ void k_add_partials(float *__restrict__ y, uint64_t ldy, const float *__restrict__ x, uint64_t ldx,
                               const float *__restrict__ part, uint64_t ldp, uint64_t pstride, int n_part,
                               uint64_t n)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int r = blockIdx.y;
    if (i >= n) return;
    float ps = part[(uint64_t)r * ldp + i];
    for (int q = 1; q < n_part; q++) ps += part[(uint64_t)q * pstride + (uint64_t)r * ldp + i];
    y[(uint64_t)r * ldy + i] = x[(uint64_t)r * ldx + i] + ps;
}

extern "C" int qgpu_add_partials(float *y, uint64_t ldy, const float *x, uint64_t ldx, const float *part,
                                 uint64_t ldp, int n_part, uint64_t n, int rows)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!y || !x || !part || n_part < 1 || n_part > 8 || rows < 1 || rows > QGPU_MAX_B || !n) return QGPU_E_ARG;
    if (rows > 1 && (ldy < n || ldx < n || ldp < n)) return QGPU_E_ARG;
    hipLaunchKernelGGL(k_add_partials, dim3((unsigned)((n + 255) / 256), (unsigned)rows), dim3(256), 0, qg::stream,
                       y, ldy, x, ldx, part, ldp, (uint64_t)rows * ldp, n_part, n);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_gemv_prepare(const float *x, uint64_t ldx, int n, uint64_t ne0)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!x || (n > 1 && ldx < ne0)) return QGPU_E_ARG;
    const qgpu_act a = copy_act(x, ldx);
    return prep_act(lib_exec(), &a, n, ne0, 1);
}

extern "C" int qgpu_act_prepare(const qgpu_act *act, int n, uint64_t ne0)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!act || !act->xout) return QGPU_E_ARG;
    return prep_act(lib_exec(), act, n, ne0, ne0 <= MAX_K ? 1 : 0);
}

extern "C" int qgpu_gemv_prepared(const qgpu_tensor *W, int n, float *out, uint64_t ldo, int flags)
{
    if (!W || !W->packed) return QGPU_E_TYPE;
    return gemv_multi(&W, 1, nullptr, n, &out, &ldo, flags, nullptr, nullptr);
}

extern "C" int qgpu_gemv_prepared_split(const qgpu_tensor *W, int n, float *part, uint64_t ldp, int ks)
{
    if (!W || !part) return QGPU_E_ARG;
    if (!W->packed) return QGPU_E_TYPE;
    if (n > 1 && ldp < W->ne1) return QGPU_E_ARG;
    return gemv_multi(&W, 1, nullptr, n, &part, &ldp, 0, nullptr, nullptr, ks);
}

extern "C" int qgpu_gemv_rows_batch(const qgpu_tensor *W, const float *x, uint64_t ldx, int n, float *out,
                                    uint64_t ldo, uint64_t r0, uint64_t r1)
{
    if (!x || !W || (n > 1 && ldx < W->ne0)) return QGPU_E_ARG;
    const qgpu_act a = copy_act(x, ldx);
    return gemv_multi(&W, 1, &a, n, &out, &ldo, 0, &r0, &r1);
}

// ---------------------------------------------------------------- dequant rows (embedding)
// Scalar dequant of whole rows, bit-exact with the reference dequant_row
// (quant.c:86-208: round-to-nearest products, no FMA), from the packed tile
// records (PK) or the GGUF row layout.
template <int FMT, int PK>
__global__ __launch_bounds__(256) void k_dequant_rows(const uint8_t *__restrict__ W, uint64_t ne0, uint64_t ne1,
                                                      const uint32_t *__restrict__ rows, float *__restrict__ out,
                                                      uint64_t ldo)
{
    const uint32_t r = rows[blockIdx.x];
    float *o = out + (uint64_t)blockIdx.x * ldo;
    const uint32_t nchunk = (uint32_t)(ne0 / 32);
    if (r >= ne1) {                                   // out-of-range id: zeros, never a wild read
        for (uint32_t i = threadIdx.x; i < ne0; i += blockDim.x) o[i] = 0.0f;
        return;
    }
    for (uint32_t c = threadIdx.x; c < nchunk; c += blockDim.x) {
        float w[32];
        if (FMT == T_IQ4_XS) {
            const uint32_t nsb = (uint32_t)(ne0 / 256), sb = c >> 3, ib = c & 7;
            const uint8_t *rec = W + ((uint64_t)(r / IQ4_TILE_ROWS) * nsb + sb) * IQ4_REC_BYTES;
            const uint32_t n = r % IQ4_TILE_ROWS;
            const uint2 hdr = *(const uint2 *)(rec + n * 8);
            const float dl = __fmul_rn(h2f(hdr.x & 0xFFFFu), (float)hdr_scale(hdr, (int)ib));
            const int8_t kv[16] = { -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t q = *(const uint32_t *)(rec + IQ4_HDR_BYTES + ((ib / 4) * 64 + g * 16 + n) * 16 + (ib % 4) * 4);
#pragma unroll
                for (int cc = 0; cc < 4; cc++) {
                    const uint32_t byte = (q >> (8 * cc)) & 0xFF;
                    w[4 * g + cc] = __fmul_rn(dl, (float)kv[byte & 15]);
                    w[16 + 4 * g + cc] = __fmul_rn(dl, (float)kv[byte >> 4]);
                }
            }
        } else if (PK) {
            const uint32_t nsb = (uint32_t)(ne0 / 256), sb = c >> 3, ib = c & 7;
            const uint8_t *rec = W + ((uint64_t)(r / IQ4_TILE_ROWS) * nsb + sb) * packed_rec_bytes(FMT);
            const int n = (int)(r % IQ4_TILE_ROWS);
            float d1 = 0.0f, m1 = 0.0f, ds0 = 0.0f, ds1 = 0.0f;
            if (FMT == T_Q4_K || FMT == T_Q5_K) {
                const uint4 h = *(const uint4 *)(rec + n * 16);
                d1 = __fmul_rn(h2f(h.x & 0xFFFFu), (float)kq_sc(h, (int)ib));
                m1 = __fmul_rn(h2f(h.x >> 16), (float)kq_m(h, (int)ib));
            } else if (FMT == T_Q6_K) {
                const float d = h2f(*(const uint16_t *)(rec + KQ_D6 + 2 * n));
                ds0 = __fmul_rn(d, (float)(int8_t)rec[n * 16 + 2 * ib]);
                ds1 = __fmul_rn(d, (float)(int8_t)rec[n * 16 + 2 * ib + 1]);
            } else {
                ds0 = h2f(*(const uint16_t *)(rec + n * 16 + 2 * ib));
            }
#pragma unroll
            for (int g = 0; g < 4; g++) {
#pragma unroll
                for (int cc = 0; cc < 4; cc++) {
                    int qa, qb;                           // elements 4g+cc and 16+4g+cc of the sub-block
                    if (FMT == T_Q8_0) {
                        const uint8_t *q = rec + KQ_Q + ((ib / 2) * 64 + g * 16 + n) * 16 + (ib & 1) * 8;
                        qa = (int8_t)q[cc];
                        qb = (int8_t)q[4 + cc];
                    } else {
                        const uint32_t byte = (*(const uint32_t *)(rec + kq_qoff(FMT, n, g, (int)ib)) >> (8 * cc)) & 0xFF;
                        qa = byte & 15;
                        qb = byte >> 4;
                        if (FMT == T_Q5_K) {
                            const uint32_t hb = rec[KQ_HB5 + (g * 16 + n) * 8 + ib];
                            qa += ((hb >> cc) & 1) << 4;
                            qb += ((hb >> (4 + cc)) & 1) << 4;
                        }
                        if (FMT == T_Q6_K) {
                            const uint32_t hb = rec[KQ_HB6 + (g * 16 + n) * 16 + (ib / 2) * 4 + cc] >> (4 * (ib & 1));
                            qa = (qa | ((hb & 3) << 4)) - 32;
                            qb = (qb | (((hb >> 2) & 3) << 4)) - 32;
                        }
                    }
                    if (FMT == T_Q4_K || FMT == T_Q5_K) {
                        w[4 * g + cc] = __fsub_rn(__fmul_rn(d1, (float)qa), m1);
                        w[16 + 4 * g + cc] = __fsub_rn(__fmul_rn(d1, (float)qb), m1);
                    } else if (FMT == T_Q6_K) {
                        w[4 * g + cc] = __fmul_rn(ds0, (float)qa);
                        w[16 + 4 * g + cc] = __fmul_rn(ds1, (float)qb);
                    } else {
                        w[4 * g + cc] = __fmul_rn(ds0, (float)qa);
                        w[16 + 4 * g + cc] = __fmul_rn(ds0, (float)qb);
                    }
                }
            }
        } else {
            const uint64_t rb = (FMT == T_F32) ? ne0 * 4 : (FMT == T_Q8_0 ? ne0 / 32 * 34 :
                                ne0 / 256 * (FMT == T_Q4_K ? 144 : FMT == T_Q5_K ? 176 : 210));
            decode_chunk<FMT>(W + (uint64_t)r * rb, c, w);
        }
#pragma unroll
        for (int j = 0; j < 32; j++) o[(uint64_t)c * 32 + j] = w[j];
    }
}

extern "C" int qgpu_dequant_rows(const qgpu_tensor *W, const uint32_t *rows, int n, float *out, uint64_t ldo)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!W || !rows || !out || n < 0 || (n > 1 && ldo < W->ne0) || W->ne0 % 32) return QGPU_E_ARG;
    if (!n) return QGPU_OK;
    const dim3 grid((unsigned)n), blk(256);
#define DQ(F, P) hipLaunchKernelGGL((k_dequant_rows<F, P>), grid, blk, 0, qg::stream, (const uint8_t *)W->data, W->ne0, W->ne1, rows, out, ldo)
#define DQ2(F) do { if (W->packed) DQ(F, 1); else DQ(F, 0); } while (0)
    switch (W->type) {
    case T_IQ4_XS: DQ(T_IQ4_XS, 1); break;
    case T_F32: DQ(T_F32, 0); break;
    case T_Q8_0: DQ2(T_Q8_0); break;
    case T_Q4_K: DQ2(T_Q4_K); break;
    case T_Q5_K: DQ2(T_Q5_K); break;
    case T_Q6_K: DQ2(T_Q6_K); break;
    default: return QGPU_E_TYPE;
    }
#undef DQ2
#undef DQ
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}
