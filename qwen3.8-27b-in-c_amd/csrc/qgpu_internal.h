// Internal declarations shared by the HIP translation units of libqgpu.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "qgpu.h"

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ4_XS = 23 };

// Packed IQ4_XS: rows grouped in tiles of 16; per (tile, super-block) one
// 2176-byte record = 16 x 8-byte row headers (d, scales_h, scales_l) followed by
// 2048 bytes of nibbles ordered for the matrix core (see gemv.hip).
#define IQ4_TILE_ROWS   16
#define IQ4_REC_BYTES   2176
#define IQ4_HDR_BYTES   128

struct qgpu_tensor {
    int      type;
    uint64_t ne0, ne1;
    void    *data;        // device bytes
    uint64_t bytes;       // device allocation size
    uint64_t algo_bytes;  // GGUF size of the matrix
    int      packed;      // 1: IQ4_XS tile layout
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
