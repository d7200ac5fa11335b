// libqgpu runtime: device selection, stream, memory, events, graphs and the
// weight registry (upload + repack).  C-ABI in include/qgpu.h.
#include <stdio.h>
#include <string.h>
#include "qgpu_internal.h"

namespace qg {
hipStream_t stream = nullptr;
int initialized = 0;
void *ws = nullptr;
size_t ws_bytes = 0;
int n_cu = 0;

int check(hipError_t e) { return e == hipSuccess ? QGPU_OK : (int)e; }

int ensure_init() { return initialized ? QGPU_OK : qgpu_init(0); }

uint64_t elems_per_block(int t)
{
    switch (t) {
    case T_F32: case T_F16: return 1;
    case T_Q8_0: return 32;
    case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_IQ4_XS: return 256;
    default: return 0;
    }
}

size_t row_bytes(int t, uint64_t ne0)
{
    uint64_t bs;
    switch (t) {
    case T_F32: bs = 4; break;
    case T_F16: bs = 2; break;
    case T_Q8_0: bs = 34; break;
    case T_Q4_K: bs = 144; break;
    case T_Q5_K: bs = 176; break;
    case T_Q6_K: bs = 210; break;
    case T_IQ4_XS: bs = 136; break;
    default: return 0;
    }
    const uint64_t e = elems_per_block(t);
    return (ne0 % e) ? 0 : (size_t)(ne0 / e * bs);
}
}  // namespace qg

// implemented in gemv.hip
int qg_repack(int type, const void *raw, uint64_t ne0, uint64_t ne1, void *packed, int unpack);
size_t qg_gemv_workspace_bytes();

extern "C" int qgpu_init(int device)
{
    if (qg::initialized) return QGPU_OK;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) return QGPU_E_INIT;
    QG_CHECK(hipSetDevice(device));
    QG_CHECK(hipDeviceGetAttribute(&qg::n_cu, hipDeviceAttributeMultiprocessorCount, device));
    QG_CHECK(hipStreamCreateWithFlags(&qg::stream, hipStreamNonBlocking));
    qg::ws_bytes = qg_gemv_workspace_bytes();
    QG_CHECK(hipMalloc(&qg::ws, qg::ws_bytes));
    QG_CHECK(hipMemset(qg::ws, 0, qg::ws_bytes));
    qg::initialized = 1;
    return QGPU_OK;
}

extern "C" int qgpu_device_info(char *name, int cap, int *n_cu, uint64_t *hbm)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    int dev = 0;
    QG_CHECK(hipGetDevice(&dev));
    hipDeviceProp_t p;
    QG_CHECK(hipGetDeviceProperties(&p, dev));
    if (name && cap > 0) snprintf(name, (size_t)cap, "%s (%s)", p.name, p.gcnArchName);
    if (n_cu) *n_cu = p.multiProcessorCount;
    if (hbm) *hbm = (uint64_t)p.totalGlobalMem;
    return QGPU_OK;
}

extern "C" const char *qgpu_strerror(int s)
{
    switch (s) {
    case QGPU_OK: return "ok";
    case QGPU_E_ARG: return "invalid argument";
    case QGPU_E_TYPE: return "unsupported ggml type";
    case QGPU_E_INIT: return "no HIP device / qgpu_init failed";
    case QGPU_E_RANGE: return "size beyond the supported maximum";
    default: return s > 0 ? hipGetErrorString((hipError_t)s) : "unknown error";
    }
}

extern "C" int qgpu_sync(void)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    return qg::check(hipStreamSynchronize(qg::stream));
}

extern "C" int qgpu_malloc(void **p, size_t bytes)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!p) return QGPU_E_ARG;
    return qg::check(hipMalloc(p, bytes ? bytes : 1));
}

// Work queued on the library stream may still read the allocation: drain the
// stream first, so a free is always safe right after an asynchronous call.
extern "C" int qgpu_free(void *p)
{
    if (!p) return QGPU_OK;
    if (qg::stream) QG_CHECK(hipStreamSynchronize(qg::stream));
    return qg::check(hipFree(p));
}

extern "C" int qgpu_memcpy_h2d(void *d, const void *s, size_t n)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    QG_CHECK(hipMemcpyAsync(d, s, n, hipMemcpyHostToDevice, qg::stream));
    return qg::check(hipStreamSynchronize(qg::stream));
}

extern "C" int qgpu_memcpy_d2h(void *d, const void *s, size_t n)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    QG_CHECK(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToHost, qg::stream));
    return qg::check(hipStreamSynchronize(qg::stream));
}

// Pinned, coherent host memory: kernels store to it through the fabric, and the host
// sees those stores without a copy or a stream synchronisation.
extern "C" int qgpu_host_malloc(void **p, size_t bytes)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!p || !bytes) return QGPU_E_ARG;
    *p = nullptr;
    return qg::check(hipHostMalloc(p, bytes, hipHostMallocDefault));
}

extern "C" int qgpu_host_free(void *p)
{
    if (!p) return QGPU_OK;
    if (qg::stream) QG_CHECK(hipStreamSynchronize(qg::stream));
    return qg::check(hipHostFree(p));
}

extern "C" int qgpu_memcpy_d2d(void *d, const void *s, size_t n)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    return qg::check(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, qg::stream));
}

extern "C" int qgpu_memset(void *d, int v, size_t n)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    return qg::check(hipMemsetAsync(d, v, n, qg::stream));
}

extern "C" int qgpu_event_create(void **ev)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    return qg::check(hipEventCreate((hipEvent_t *)ev));
}
extern "C" int qgpu_event_destroy(void *ev) { return qg::check(hipEventDestroy((hipEvent_t)ev)); }
extern "C" int qgpu_event_record(void *ev) { return qg::check(hipEventRecord((hipEvent_t)ev, qg::stream)); }
extern "C" int qgpu_event_elapsed_ms(void *a, void *b, float *ms)
{
    QG_CHECK(hipEventSynchronize((hipEvent_t)b));
    return qg::check(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
}

extern "C" int qgpu_graph_begin(void)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    return qg::check(hipStreamBeginCapture(qg::stream, hipStreamCaptureModeThreadLocal));
}

extern "C" int qgpu_graph_end(void **exec)
{
    hipGraph_t g;
    QG_CHECK(hipStreamEndCapture(qg::stream, &g));
    hipGraphExec_t e;
    hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    QG_CHECK(err);
    *exec = (void *)e;
    return QGPU_OK;
}

extern "C" int qgpu_graph_launch(void *exec) { return qg::check(hipGraphLaunch((hipGraphExec_t)exec, qg::stream)); }
extern "C" int qgpu_graph_destroy(void *exec) { return qg::check(hipGraphExecDestroy((hipGraphExec_t)exec)); }

// ------------------------------------------------------------------ weights
static int make_tensor(const void *dev_raw, int type, uint64_t ne0, uint64_t ne1, qgpu_tensor **out)
{
    const size_t rb = qg::row_bytes(type, ne0);
    if (!out || !ne0 || !ne1 || !rb) return type == T_F16 || !qg::elems_per_block(type) ? QGPU_E_TYPE : QGPU_E_ARG;
    if (type == T_F16) return QGPU_E_TYPE;
    qgpu_tensor *t = new qgpu_tensor();
    t->type = type; t->ne0 = ne0; t->ne1 = ne1;
    t->algo_bytes = (uint64_t)rb * ne1;
    if (packed_rec_bytes(type) && ne0 % 256 == 0) {        // matrix-core tile records
        const uint64_t tiles = (ne1 + IQ4_TILE_ROWS - 1) / IQ4_TILE_ROWS;
        t->bytes = tiles * (ne0 / 256) * packed_rec_bytes(type);
        t->packed = 1;
        hipError_t e = hipMalloc(&t->data, t->bytes);
        if (e != hipSuccess) { delete t; return (int)e; }
        int rc = qg_repack(type, dev_raw, ne0, ne1, t->data, 0);
        if (rc) { (void)hipFree(t->data); delete t; return rc; }
    } else {
        t->bytes = t->algo_bytes;
        hipError_t e = hipMalloc(&t->data, t->bytes);
        if (e == hipSuccess) e = hipMemcpyAsync(t->data, dev_raw, t->bytes, hipMemcpyDeviceToDevice, qg::stream);
        if (e != hipSuccess) { (void)hipFree(t->data); delete t; return (int)e; }
    }
    *out = t;
    return QGPU_OK;
}

extern "C" int qgpu_tensor_from_device(const void *dev, int type, uint64_t ne0, uint64_t ne1, qgpu_tensor **out)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!dev) return QGPU_E_ARG;
    return make_tensor(dev, type, ne0, ne1, out);
}

extern "C" int qgpu_tensor_upload(const void *host, int type, uint64_t ne0, uint64_t ne1, qgpu_tensor **out)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    const size_t rb = qg::row_bytes(type, ne0);
    if (!host || !rb || !ne1) return rb ? QGPU_E_ARG : QGPU_E_TYPE;
    const size_t n = rb * ne1;
    void *tmp = nullptr;
    QG_CHECK(hipMalloc(&tmp, n));
    hipError_t e = hipMemcpyAsync(tmp, host, n, hipMemcpyHostToDevice, qg::stream);
    if (e != hipSuccess) { (void)hipFree(tmp); return (int)e; }
    rc = make_tensor(tmp, type, ne0, ne1, out);
    hipError_t s = hipStreamSynchronize(qg::stream);
    (void)hipFree(tmp);
    if (rc) return rc;
    return qg::check(s);
}

extern "C" int qgpu_tensor_free(qgpu_tensor *t)
{
    if (!t) return QGPU_OK;
    hipError_t e = hipFree(t->data);
    delete t;
    return qg::check(e);
}

extern "C" int qgpu_tensor_download(const qgpu_tensor *t, void *host)
{
    int rc = qg::ensure_init();
    if (rc) return rc;
    if (!t || !host) return QGPU_E_ARG;
    if (!t->packed) return qgpu_memcpy_d2h(host, t->data, t->algo_bytes);
    void *tmp = nullptr;
    QG_CHECK(hipMalloc(&tmp, t->algo_bytes));
    rc = qg_repack(t->type, tmp, t->ne0, t->ne1, t->data, 1);
    if (!rc) rc = qgpu_memcpy_d2h(host, tmp, t->algo_bytes);
    (void)hipFree(tmp);
    return rc;
}

extern "C" int qgpu_tensor_shape(const qgpu_tensor *t, int *type, uint64_t *ne0, uint64_t *ne1)
{
    if (!t) return QGPU_E_ARG;
    if (type) *type = t->type;
    if (ne0) *ne0 = t->ne0;
    if (ne1) *ne1 = t->ne1;
    return QGPU_OK;
}

extern "C" uint64_t qgpu_tensor_bytes(const qgpu_tensor *t) { return t ? t->algo_bytes : 0; }
