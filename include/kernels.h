/*
 * kernels.h -- GEMV and elementwise ops on HOST pointers, computed on the GPU.
 *
 * Drop-in for the reference interface include/kernels.h:1-46 (same names,
 * arguments and semantics; synchronous: results are valid on return).  Each
 * call stages x into device memory, runs the HIP kernel (include/qgpu.h) and
 * copies the result back, so the rates include PCIe transfers; the model
 * runtime uses the device-pointer entry points of qgpu.h directly.  A weight
 * tensor is uploaded (and, for IQ4_XS, repacked) the first time it is used and
 * cached by its data address until kernels_release_weights().
 */
#if !defined(QWEN_KERNELS_H) && !defined(KERNELS_H)   /* either header, whichever came first */
#define QWEN_KERNELS_H
/* the reference header of the same name is superseded by this one when both
   are on the include path (reference drivers compiled against this library) */
#define KERNELS_H

#include "gguf.h"
#include "threadpool.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GEMV_MAX_B 8

/* out[r] = dot(x, row r of W) for r in [r0, r1) (reference kernels.c:298-321) */
void gemv_rows(const gguf_tensor_info_t *W, const float *x, float *out, uint64_t r0, uint64_t r1);
/* all rows (kernels.c:615-621) */
void gemv(pool_t *pool, const gguf_tensor_info_t *W, const float *x, float *out);
/* out[t*ldo + r] = dot(x[t*ldx ...], row r) for t < n <= 8 (kernels.c:570-648) */
void gemv_rows_batch(const gguf_tensor_info_t *W, const float *x, uint64_t ldx, int n,
                     float *out, uint64_t ldo, uint64_t r0, uint64_t r1);
void gemv_batch(pool_t *pool, const gguf_tensor_info_t *W, const float *x, uint64_t ldx, int n,
                float *out, uint64_t ldo);
/* several matrices sharing x (kernels.c:666-736) */
void gemv_multi(pool_t *pool, const gguf_tensor_info_t *const *Ws, const float *x, float *const *outs, int n_mat);
void gemv_multi_batch(pool_t *pool, const gguf_tensor_info_t *const *Ws, const float *x, uint64_t ldx, int n,
                      float *const *outs, const uint64_t *ldos, int n_mat);

/* ops (kernels.c:741-939) */
void rmsnorm(float *out, const float *x, const float *weight, uint64_t n, float eps);
void l2norm(float *out, const float *x, uint64_t n, float eps);
void silu_inplace(float *x, uint64_t n);
void sigmoid_inplace(float *x, uint64_t n);
void softplus_inplace(float *x, uint64_t n);
void softmax_inplace(float *x, uint64_t n);

/* frees the device copies of weights uploaded by the calls above */
void kernels_release_weights(void);
/* first failure of the calls above (0 = none): an unsupported weight type,
 * a batch above 8, rows past the matrix, or a device error.  The failing call
 * wrote zeros to its outputs, as the reference does for unsupported types
 * (kernels.c:596).  No reference counterpart. */
int kernels_status(void);

#ifdef __cplusplus
}
#endif
#endif
