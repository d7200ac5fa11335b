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

namespace qg {
extern hipStream_t stream;
extern int initialized;
// workspace for the GEMV activation prep (digit planes + scales)
extern void *ws;
extern size_t ws_bytes;
int ensure_init();
int check(hipError_t e);
size_t row_bytes(int type, uint64_t ne0);
uint64_t elems_per_block(int type);
}  // namespace qg

#define QG_CHECK(expr) do { hipError_t _e = (expr); if (_e != hipSuccess) return (int)_e; } while (0)
#define QG_LAUNCH_CHECK() do { hipError_t _e = hipGetLastError(); if (_e != hipSuccess) return (int)_e; } while (0)
