// Internal declarations shared by the HIP translation units of libqgpu.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "qgpu.h"

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ4_XS = 23 };

// Packed matrices: rows grouped in tiles of 16; per (tile, 256-column
// super-block) one record holding the 16 row slices, ordered for the matrix
// core (see gemv.hip).  The record is as large as the 16 GGUF row slices.
//   IQ4_XS 2176 = 16 x 8 B headers (d, scales) + 2048 B nibbles
//   Q4_K   2304 = 16 x 16 B headers (d, dmin, 6-bit scales and mins) + 2048 B nibbles
//   Q5_K   2816 = Q4_K + 512 B fifth bits
//   Q6_K   3360 = 16 x 16 B int8 scales + 16 x 2 B d + 2048 B low nibbles + 1024 B high bit pairs
//   Q8_0   4352 = 16 x 8 fp16 d + 4096 B int8 quants
#define IQ4_TILE_ROWS   16
#define IQ4_REC_BYTES   2176
#define IQ4_HDR_BYTES   128
static inline __host__ __device__ uint32_t packed_rec_bytes(int type)
{
    switch (type) {
    case T_IQ4_XS: return 2176;
    case T_Q4_K: return 2304;
    case T_Q5_K: return 2816;
    case T_Q6_K: return 3360;
    case T_Q8_0: return 4352;
    default: return 0;
    }
}

struct qgpu_tensor {
    int      type;
    uint64_t ne0, ne1;
    void    *data;        // device bytes
    uint64_t bytes;       // device allocation size
    uint64_t algo_bytes;  // GGUF size of the matrix
    int      packed;      // 1: tile records (IQ4_XS, Q4_K, Q5_K, Q6_K, Q8_0 with ne0 % 256 == 0)
};

// State that only a later step reads (GDN state and conv snapshots, new KV
// cache rows) goes out with non-temporal stores: it leaves this XCD's L2 as it
// is written instead of in the write-back at the end of the kernel, which
// otherwise holds up the next launch.  Results the next launch reads stay
// plain stores (non-temporal ones made those reads slower).
typedef float qg_v4f __attribute__((ext_vector_type(4)));
static __device__ __forceinline__ void st_stream4(float *p, float a, float b, float c, float d)
{
    __builtin_nontemporal_store(qg_v4f{a, b, c, d}, (qg_v4f *)p);
}
static __device__ __forceinline__ void st_stream4(float *p, float4 v) { st_stream4(p, v.x, v.y, v.z, v.w); }

// GEMV activation workspace (qg::ws): two digit planes of 4 tokens each, then
// their conversion factors, then the deferred-RMSNorm sums (gemv.hip).
#define MAX_K       65536
#define MAX_NSB     (MAX_K / 256)
#define DIGIT_TILE  3072     // digit bytes of one (4-token plane, super-block): 4 tokens x 3 digits x 256
#define DIGIT_SUB   768      // of one pair of sub-blocks
#define PLANE_BYTES ((size_t)MAX_NSB * DIGIT_TILE)
#define XS_FLOATS   ((size_t)MAX_NSB * 16)

// Lane reductions with DPP moves (VALU, no LDS round trip).  A 16-lane row: lane ^ 1, lane ^ 2
// (quad_perm), the other quad of the half row (row_half_mirror), the other half row
// (row_mirror); each step combines a value with its mirror image, so every lane of the row ends
// with the same bits.  A wave: the four row results read from lanes 0, 16, 32, 48, combined in a
// fixed order (every lane of the wave gets the same bits).  All 64 lanes must be active.
template <int CTRL>
static __device__ __forceinline__ float dpp_mov(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
static __device__ __forceinline__ float rowsum16(float v)
{
    v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);   // row_half_mirror
    v += dpp_mov<0x140>(v);   // row_mirror
    return v;
}
static __device__ __forceinline__ float rowmax16(float v)
{
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return v;
}
static __device__ __forceinline__ float lane_value(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
static __device__ __forceinline__ float wave_sum64(float v)
{
    v = rowsum16(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
static __device__ __forceinline__ float wave_max64(float v)
{
    v = rowmax16(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Digit planes of one (4-token plane, 256-element super-block), written by a
// block of 256 threads: thread e holds element e of the super-block for the 4
// tokens (v[i]; tokens past the batch hold 0) and m[i], the largest |v[i]| of
// its wave.  Per token t the shift s_t puts the super-block maximum just under
// 2^22 (s_t = 22 - exponent of the max; 0 for an all-zero or non-finite max);
// x 2^s_t rounds to an integer X split into three balanced base-256 digits (X =
// d0 + 2^8 d1 + 2^16 d2, d0, d1 in [-128, 127], |d2| <= 64): x to 2^-23 of the
// super-block maximum.  A tile layout (3072 bytes): lane l = g*16 + m of the
// GEMV wave holds, for A row m = t*4 + dgt (token-major; rows with dgt = 3 are
// zero), digit dgt of token t at the 8 elements of sub-block ib that K-slots
// 8g..8g+7 stand for (slot 8g+c, c < 4 -> element 4g+c; slot 8g+4+c -> element
// 16+4g+c); two sub-blocks interleave so a lane fetches 16 bytes, and each
// token's lanes come first to last in one 192-byte run: byte
// (ib/2)*768 + (t*12 + g*3 + dgt)*16 + (ib%2)*8 + slot%8.  A GEMV of fewer than
// 4 tokens reads only the runs of its tokens.  xs_tile[dgt*4 + t] =
// 2^(8 dgt - s_t) converts the integer result of A row t*4 + dgt.  Every thread of the block calls it (two
// barriers); in blocks of more than 256 threads, threads 0..255 pass active =
// true and the others false (they only take part in the barriers).
struct ActDigitLds {
    uint8_t stage[DIGIT_TILE];
    float mx[4][4];          // [token][wave]
};
static __device__ __forceinline__ void act_digits(const float v[4], const float m[4], ActDigitLds &L,
                                                  uint8_t *__restrict__ A_tile, float *__restrict__ xs_tile,
                                                  bool active = true)
{
    const int e = threadIdx.x & 255, lane = e & 63, wv = e >> 6;
    if (active && lane == 0)
#pragma unroll
        for (int i = 0; i < 4; i++) L.mx[i][wv] = m[i];
    __syncthreads();
    int shift[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float mx = fmaxf(fmaxf(L.mx[i][0], L.mx[i][1]), fmaxf(L.mx[i][2], L.mx[i][3]));
        int E = 0;
        if (mx > 0.0f && isfinite(mx)) { frexpf(mx, &E); shift[i] = 22 - E; }
        else shift[i] = 0;
    }
    if (active) {
        const int ib = e >> 5, w = e & 31, up = w >> 4, jj = w & 15, gg = jj >> 2, c = jj & 3;
        const int boff = (ib >> 1) * DIGIT_SUB + (ib & 1) * 8 + up * 4 + c;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float sv = ldexpf(v[i], shift[i]);
            int X = isfinite(sv) ? (int)rintf(sv) : 0;
#pragma unroll
            for (int dg = 0; dg < 3; dg++) {
                const int d = (dg < 2) ? (int)(int8_t)(X & 0xFF) : X;     // balanced base-256 digit
                X = (X - d) >> 8;
                L.stage[boff + (i * 12 + gg * 3 + dg) * 16] = (uint8_t)d;
            }
        }
    }
    __syncthreads();
    if (active) {
        if (e < DIGIT_TILE / 16) ((uint4 *)A_tile)[e] = ((const uint4 *)L.stage)[e];
        if (e < 16) xs_tile[e] = ldexpf(1.0f, 8 * (e >> 2) - shift[e & 3]);
    }
}

// Digits of one token of a super-block, written by a block of 256 threads: thread e holds element
// e of the super-block (v) and mx, the super-block's largest |v| (the same value in every thread).
// Wave r holds elements 64r..64r+63, which are the token's whole 192-byte run of sub-block pair r
// in the digit tile (layout above act_digits): lane l = 16h + 4gg + c holds element 64r + 16h +
// 4gg + c, whose digit dg is byte r*768 + i*192 + gg*48 + dg*16 + 4h + c (i: the token's slot in
// its 4-token plane).  The four lanes of a quad hold the four bytes of one dword per digit; a byte
// transpose inside the quad (DPP broadcasts and two v_perm_b32) gives lane c the dword of digit c,
// and lanes c < 3 store it -- no staging through LDS.  The shift and digits are those act_digits
// computes for the same token and maximum.
static __device__ __forceinline__ void tok_digits(float v, float mx, int i, uint8_t *__restrict__ A_tile,
                                                  float *__restrict__ xs_tile)
{
    const int e = threadIdx.x & 255, lane = e & 63, wv = e >> 6;
    // shift puts the super-block maximum just under 2^22 (0 for an all-zero or non-finite maximum)
    int shift = 0;
    if (mx > 0.0f && isfinite(mx)) {
        int E;
        frexpf(mx, &E);
        shift = 22 - E;
    }
    // three balanced base-256 digits of X = rint(v 2^shift), packed in bytes 0..2 of P
    const float sv = ldexpf(v, shift);
    int X = isfinite(sv) ? (int)rintf(sv) : 0;
    uint32_t P = 0;
#pragma unroll
    for (int dg = 0; dg < 3; dg++) {
        const int d = (dg < 2) ? (int)(int8_t)(X & 0xFF) : X;
        X = (X - d) >> 8;
        P |= ((uint32_t)d & 0xFFu) << (8 * dg);
    }
    // quad byte transpose: lane c gets byte c of P from each lane of its quad, in lane order
    const uint32_t c = (uint32_t)lane & 3u;
    const uint32_t P0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)P, 0x00, 0xF, 0xF, false);
    const uint32_t P1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)P, 0x55, 0xF, 0xF, false);
    const uint32_t P2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)P, 0xAA, 0xF, 0xF, false);
    const uint32_t P3 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)P, 0xFF, 0xF, 0xF, false);
    // v_perm_b32 selectors: 0..3 bytes of the second operand, 4..7 of the first, 12 the constant 0
    const uint32_t W = __builtin_amdgcn_perm(P1, P0, c | ((c + 4u) << 8) | 0x0C0C0000u) |
                       __builtin_amdgcn_perm(P3, P2, 0x00000C0Cu | (c << 16) | ((c + 4u) << 24));
    uint8_t *tile = A_tile + wv * DIGIT_SUB + i * 192;
    if (c < 3) *(uint32_t *)(tile + ((lane >> 2) & 3) * 48 + c * 16 + (lane >> 4) * 4) = W;
    if (e < 4) xs_tile[4 * e + i] = ldexpf(1.0f, 8 * e - shift);
}

namespace qg {
extern hipStream_t stream;
extern int initialized;
// workspace for the GEMV activation prep (digit planes + scales)
extern void *ws;
extern size_t ws_bytes;
extern int n_cu;          // compute units of the device

int ensure_init();
int check(hipError_t e);
size_t row_bytes(int type, uint64_t ne0);
uint64_t elems_per_block(int type);
}  // namespace qg

#define QG_CHECK(expr) do { hipError_t _e = (expr); if (_e != hipSuccess) return (int)_e; } while (0)
#define QG_LAUNCH_CHECK() do { hipError_t _e = hipGetLastError(); if (_e != hipSuccess) return (int)_e; } while (0)
