// Norms, activations, residual add and greedy argmax (gfx950).
// Row-parallel kernels: one 256-thread block per row, fp32 throughout.
// The reference's own results differ from these only by fp32 rounding
// (its AVX2 exp is a degree-7 Taylor polynomial, kernels.c:807-822; here the
// device libm expf is used).
#include "qgpu_internal.h"

namespace qg {
void *ws_small = nullptr;     // 128 KiB: argmax partials (64 rows x AMAX_CHUNKS keys)
}

static __device__ __forceinline__ float block_sum(float v, float *sh)
{
#pragma unroll
    for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += sh[i];
    return s;
}

static __device__ __forceinline__ float block_max(float v, float *sh)
{
#pragma unroll
    for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    float s = sh[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) s = fmaxf(s, sh[i]);
    return s;
}

__global__ __launch_bounds__(256) void k_rmsnorm(float *out, uint64_t ldo, const float *x, uint64_t ldx,
                                                 const float *w, uint64_t n, float eps)
{
    __shared__ float sh[4];
    const float *xr = x + (uint64_t)blockIdx.x * ldx;
    float *orow = out + (uint64_t)blockIdx.x * ldo;
    float s = 0.0f;
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) s = fmaf(xr[i], xr[i], s);
    s = block_sum(s, sh);
    const float scale = 1.0f / sqrtf(s / (float)n + eps);
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) orow[i] = w ? (xr[i] * scale) * w[i] : xr[i] * scale;
}

__global__ __launch_bounds__(256) void k_l2norm(float *out, uint64_t ldo, const float *x, uint64_t ldx,
                                                uint64_t n, float eps)
{
    __shared__ float sh[4];
    const float *xr = x + (uint64_t)blockIdx.x * ldx;
    float *orow = out + (uint64_t)blockIdx.x * ldo;
    float s = 0.0f;
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) s = fmaf(xr[i], xr[i], s);
    s = block_sum(s, sh);
    const float nr = sqrtf(s);
    const float scale = 1.0f / (nr > eps ? nr : eps);
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) orow[i] = xr[i] * scale;
}

__global__ void k_unary(float *x, uint64_t n, int op)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r;
    if (op == 0) r = v / (1.0f + expf(-v));                              // silu
    else if (op == 1) r = 1.0f / (1.0f + expf(-v));                      // sigmoid
    else r = v > 30.0f ? v : (v < -30.0f ? expf(v) : log1pf(expf(v)));   // softplus (kernels.c:874-885)
    x[i] = r;
}

__global__ __launch_bounds__(256) void k_softmax(float *x, uint64_t ld, uint64_t n)
{
    __shared__ float sh[4];
    float *r = x + (uint64_t)blockIdx.x * ld;
    float m = -INFINITY;
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, r[i]);
    m = block_max(m, sh);
    float s = 0.0f;
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float e = expf(r[i] - m);
        r[i] = e;
        s += e;
    }
    s = block_sum(s, sh);
    const float inv = 1.0f / s;
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) r[i] *= inv;
}

__global__ void k_silu_mul(float *a, uint64_t lda, const float *b, uint64_t ldb, uint64_t n)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float *ar = a + (uint64_t)blockIdx.y * lda;
    const float v = ar[i];
    ar[i] = (v / (1.0f + expf(-v))) * b[(uint64_t)blockIdx.y * ldb + i];
}

__global__ void k_add(float *y, uint64_t ldy, const float *x, uint64_t ldx, uint64_t n)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    y[(uint64_t)blockIdx.y * ldy + i] += x[(uint64_t)blockIdx.y * ldx + i];
}

// ---------------------------------------------------------------- argmax
#define AMAX_CHUNKS 256
// key = order-preserving float bits << 32 | ~index : the max key is the max
// value with the lowest index (model.c:750 strict '>').
static __device__ __forceinline__ uint64_t akey(float v, uint32_t i)
{
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (0xFFFFFFFFu - i);
}

// AMAX_CHUNKS blocks per row; a thread issues its (up to 4) loads of a pass before
// comparing, so a 248,320-logit row costs one load latency.
__global__ __launch_bounds__(256) void k_argmax_part(const float *logits, uint64_t ld, uint32_t n, uint64_t *part)
{
    __shared__ uint64_t sh[4];
    const float *r = logits + (uint64_t)blockIdx.y * ld;
    const uint32_t per = (n + AMAX_CHUNKS - 1) / AMAX_CHUNKS;
    const uint32_t lo = blockIdx.x * per, hi = min(n, lo + per);
    uint64_t best = 0;
    for (uint32_t i0 = lo + threadIdx.x; i0 < hi; i0 += 4 * 256) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = i0 + j * 256 < hi ? r[i0 + j * 256] : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (i0 + j * 256 < hi) {
                const uint64_t k = akey(v[j], i0 + j * 256);
                best = k > best ? k : best;
            }
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) {
        const uint64_t k = __shfl_xor(best, o);
        best = k > best ? k : best;
    }
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = sh[0];
        for (int i = 1; i < 4; i++) b = sh[i] > b ? sh[i] : b;
        part[(uint64_t)blockIdx.y * AMAX_CHUNKS + blockIdx.x] = b;
    }
}

__global__ void k_argmax_final(const uint64_t *part, uint32_t *out)
{
    uint64_t b = 0;
#pragma unroll
    for (int j = 0; j < AMAX_CHUNKS / 64; j++) {
        const uint64_t k = part[(uint64_t)blockIdx.x * AMAX_CHUNKS + threadIdx.x + 64 * j];
        b = k > b ? k : b;
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) {
        const uint64_t k = __shfl_xor(b, o);
        b = k > b ? k : b;
    }
    if (threadIdx.x == 0) out[blockIdx.x] = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu);
}

__global__ void k_copy(uint4 *__restrict__ d, const uint4 *__restrict__ s, uint64_t n16)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
        d[i] = s[i];
}

__global__ void k_set_i32(int *dst, int v) { *dst = v; }

// XOR of the 32-bit words of block b's grid-stride share of n16 16-byte words
// into part[b]: 4 loads in flight per thread, one plain store per block (no
// atomics: one address hit by every block serialises across the XCDs).
#define CSUM_UNROLL 4
__global__ __launch_bounds__(256) void k_checksum(const uint4 *__restrict__ s, uint64_t n16, uint32_t *part)
{
    const uint64_t nth = (uint64_t)gridDim.x * blockDim.x;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (CSUM_UNROLL - 1) * nth < n16; i += CSUM_UNROLL * nth) {
        uint4 v[CSUM_UNROLL];
#pragma unroll
        for (int u = 0; u < CSUM_UNROLL; u++) v[u] = s[i + u * nth];
#pragma unroll
        for (int u = 0; u < CSUM_UNROLL; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += nth) { const uint4 v = s[i]; acc ^= v.x ^ v.y ^ v.z ^ v.w; }
#pragma unroll
    for (int o = 32; o; o >>= 1) acc ^= __shfl_xor(acc, o);
    __shared__ uint32_t wsum[4];
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = wsum[0] ^ wsum[1] ^ wsum[2] ^ wsum[3];
}

// pos0 / cur0 >= 0: the incoming position and ring slot as values (no launch to set them first);
// otherwise they are read from *pos / *cur
// Acceptance (thread 0); with row_out, the block then copies row j of `rows` (the
// re-anchor's hidden state).  tok_out / cand0_out are written after every read of
// cand, so cand0_out may point into cand; out[0] is written last, after a system-scope
// fence (out may be host memory that the host polls).
__global__ void k_spec_accept(const uint32_t *cand, const uint32_t *vtok, int k, int force_j, int pos0, int cur0,
                              int *pos, int *cur, int nslot, uint32_t *out, const float *rows, uint64_t ld, int n,
                              float *row_out, uint32_t *tok_out, uint32_t *cand0_out)
{
    __shared__ int sj;
    if (threadIdx.x == 0) {
        int j = k;
        if (force_j >= 0)
            j = force_j < k ? force_j : k;
        else
            for (int i = 0; i < k; i++)
                if (vtok[i] != cand[i + 1]) { j = i; break; }
        for (int i = 0; i <= j; i++) out[1 + i] = cand[i];
        const uint32_t next = vtok[j], anchor = cand[j];
        out[j + 2] = next;
        if (tok_out) *tok_out = anchor;
        if (cand0_out) *cand0_out = next;
        const int c = cur0 >= 0 ? cur0 : *cur, p = pos0 >= 0 ? pos0 : *pos;
        *cur = (c + 1 + j) % nslot;
        *pos = p + j + 1;
        sj = j;
        // j last: a host polling out[0] in host memory then finds out[1 .. j+2] written
        __threadfence_system();
        out[0] = (uint32_t)j;
    }
    if (!row_out) return;
    __syncthreads();
    const float *src = rows + (uint64_t)sj * ld;
    for (int i = threadIdx.x; i < n; i += blockDim.x) row_out[i] = src[i];
}

// ---------------------------------------------------------------- C-ABI
extern "C" int qgpu_set_i32(int *dst, int value)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!dst) return QGPU_E_ARG;
    hipLaunchKernelGGL(k_set_i32, dim3(1), dim3(1), 0, qg::stream, dst, value);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_spec_accept(const uint32_t *cand, const uint32_t *vtok, int k, int force_j, int *pos, int *cur,
                                int nslot, uint32_t *out)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!cand || !vtok || !pos || !cur || !out || k < 0 || k > 15 || nslot < k + 2) return QGPU_E_ARG;
    hipLaunchKernelGGL(k_spec_accept, dim3(1), dim3(1), 0, qg::stream, cand, vtok, k, force_j, -1, -1, pos, cur,
                       nslot, out, nullptr, 0, 0, nullptr, nullptr, nullptr);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_spec_accept_at(const uint32_t *cand, const uint32_t *vtok, int k, int force_j, int pos0,
                                   int cur0, int *pos, int *cur, int nslot, uint32_t *out)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!cand || !vtok || !pos || !cur || !out || k < 0 || k > 15 || nslot < k + 2 || pos0 < 0 || cur0 < 0 ||
        cur0 >= nslot)
        return QGPU_E_ARG;
    hipLaunchKernelGGL(k_spec_accept, dim3(1), dim3(1), 0, qg::stream, cand, vtok, k, force_j, pos0, cur0, pos, cur,
                       nslot, out, nullptr, 0, 0, nullptr, nullptr, nullptr);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_spec_accept_anchor(const uint32_t *cand, const uint32_t *vtok, int k, int force_j, int pos0,
                                       int cur0, int *pos, int *cur, int nslot, uint32_t *out, const float *rows,
                                       uint64_t ld, int n, float *row_out, uint32_t *tok_out, uint32_t *cand0_out)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!cand || !vtok || !pos || !cur || !out || k < 0 || k > 15 || nslot < k + 2 || pos0 < 0 || cur0 < 0 ||
        cur0 >= nslot)
        return QGPU_E_ARG;
    if (row_out && (!rows || n < 1 || ld < (uint64_t)n)) return QGPU_E_ARG;
    hipLaunchKernelGGL(k_spec_accept, dim3(1), dim3(row_out ? 256 : 1), 0, qg::stream, cand, vtok, k, force_j, pos0,
                       cur0, pos, cur, nslot, out, rows, ld, row_out ? n : 0, row_out, tok_out, cand0_out);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_copy(void *dst, const void *src, size_t bytes)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!dst || !src || bytes % 16 || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15)) return QGPU_E_ARG;
    if (!bytes) return QGPU_OK;
    const uint64_t n16 = bytes / 16;
    const unsigned grid = (unsigned)(n16 / 256 < 8192 ? (n16 + 255) / 256 : 8192);
    hipLaunchKernelGGL(k_copy, dim3(grid), dim3(256), 0, qg::stream, (uint4 *)dst, (const uint4 *)src, n16);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

// n blocks of 256 threads.  Measured on MI355X (graph replays, 12 rotating
// 47.7 MB buffers): n = 8192 reads 47.7 MB in 8.7 us, n = 2048 in 9.6 us.
extern "C" int qgpu_checksum(const void *src, size_t bytes, uint32_t *partials, int n)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!src || !partials || bytes % 16 || ((uintptr_t)src & 15) || n < 1 || n > 65536) return QGPU_E_ARG;
    hipLaunchKernelGGL(k_checksum, dim3((unsigned)n), dim3(256), 0, qg::stream, (const uint4 *)src,
                       (uint64_t)(bytes / 16), partials);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_tensor_checksum(const qgpu_tensor *t, uint32_t *partials, int n)
{
    if (!t) return QGPU_E_ARG;
    if (t->bytes % 16) return QGPU_E_RANGE;
    return qgpu_checksum(t->data, t->bytes, partials, n);
}

extern "C" uint64_t qgpu_tensor_device_bytes(const qgpu_tensor *t) { return t ? t->bytes : 0; }

static int ensure_small()
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!qg::ws_small) QG_CHECK(hipMalloc(&qg::ws_small, 64 * AMAX_CHUNKS * sizeof(uint64_t)));
    return QGPU_OK;
}

extern "C" int qgpu_rmsnorm(float *out, uint64_t ldo, const float *x, uint64_t ldx, const float *w, uint64_t n,
                            int rows, float eps)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!out || !x || !n || rows < 0) return QGPU_E_ARG;
    if (!rows) return QGPU_OK;
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(256), 0, qg::stream, out, ldo, x, ldx, w, n, eps);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_l2norm(float *out, uint64_t ldo, const float *x, uint64_t ldx, uint64_t n, int rows, float eps)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!out || !x || !n || rows < 0) return QGPU_E_ARG;
    if (!rows) return QGPU_OK;
    hipLaunchKernelGGL(k_l2norm, dim3(rows), dim3(256), 0, qg::stream, out, ldo, x, ldx, n, eps);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

static int unary(float *x, uint64_t n, int op)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!x) return QGPU_E_ARG;
    if (!n) return QGPU_OK;
    hipLaunchKernelGGL(k_unary, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, qg::stream, x, n, op);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}
extern "C" int qgpu_silu(float *x, uint64_t n) { return unary(x, n, 0); }
extern "C" int qgpu_sigmoid(float *x, uint64_t n) { return unary(x, n, 1); }
extern "C" int qgpu_softplus(float *x, uint64_t n) { return unary(x, n, 2); }

extern "C" int qgpu_softmax(float *x, uint64_t ld, uint64_t n, int rows)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!x || rows < 0) return QGPU_E_ARG;
    if (!rows || !n) return QGPU_OK;
    hipLaunchKernelGGL(k_softmax, dim3(rows), dim3(256), 0, qg::stream, x, ld, n);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_silu_mul(float *a, uint64_t lda, const float *b, uint64_t ldb, uint64_t n, int rows)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!a || !b || rows < 0) return QGPU_E_ARG;
    if (!rows || !n) return QGPU_OK;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256), rows), dim3(256), 0, qg::stream, a, lda, b, ldb, n);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_add(float *y, uint64_t ldy, const float *x, uint64_t ldx, uint64_t n, int rows)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!y || !x || rows < 0) return QGPU_E_ARG;
    if (!rows || !n) return QGPU_OK;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((n + 255) / 256), rows), dim3(256), 0, qg::stream, y, ldy, x, ldx, n);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}

extern "C" int qgpu_argmax(const float *logits, uint64_t ld, uint32_t n, int rows, uint32_t *out)
{
    int rc = ensure_small();
    if (rc) return rc;
    if (!logits || !out || !n || rows < 0 || rows > 64) return rows > 64 ? QGPU_E_RANGE : QGPU_E_ARG;
    if (!rows) return QGPU_OK;
    uint64_t *part = (uint64_t *)qg::ws_small;
    hipLaunchKernelGGL(k_argmax_part, dim3(AMAX_CHUNKS, rows), dim3(256), 0, qg::stream, logits, ld, n, part);
    QG_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(64), 0, qg::stream, (const uint64_t *)part, out);
    QG_LAUNCH_CHECK();
    return QGPU_OK;
}
