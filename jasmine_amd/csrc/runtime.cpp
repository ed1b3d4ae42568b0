// Runtime part of the C ABI: device selection, library stream, memory, errors, RNG fill.
// Storage behind jasmine's mat_t (mat_t.hpp:53-69 allocate+zero, :30-42 release).
#include "jas_common.hpp"

#include <mutex>

namespace jas {

static thread_local std::string g_err;
static hipStream_t g_stream = nullptr;
static int g_device = -1;
static std::mutex g_init_mu;

void set_error(const std::string &msg) { g_err = msg; }

jas_status fail(jas_status code, const std::string &msg)
{
    g_err = msg;
    return code;
}

// Library-internal scratch for multi-pass kernels (partials of whole-matrix reductions).
// Grows on demand; calls on one stream are ordered, so reuse between calls is safe.
static void *g_ws = nullptr;
static size_t g_ws_bytes = 0;
void *workspace(size_t bytes, hipStream_t s)
{
    if (bytes <= g_ws_bytes) return g_ws;
    if (g_ws) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(g_ws);
    }
    size_t nb = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (hipMalloc(&g_ws, nb) != hipSuccess) {
        g_ws = nullptr;
        g_ws_bytes = 0;
        return nullptr;
    }
    g_ws_bytes = nb;
    return g_ws;
}

hipStream_t stream_or_default(jas_stream_t s)
{
    if (s) return (hipStream_t)s;
    if (!g_stream) jas_init(-1);
    return g_stream;
}

} // namespace jas

using namespace jas;

extern "C" {

const char *jas_last_error(void) { return g_err.c_str(); }
const char *jas_version(void) { return "jasmine-mi355x 0.1 (gfx950)"; }

jas_status jas_init(int device)
{
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (device < 0) device = g_device >= 0 ? g_device : 0;
    int n = 0;
    JAS_HIP(hipGetDeviceCount(&n));
    JAS_CHECK(device < n, JAS_ERR_INVALID, "jas_init: no such device");
    JAS_HIP(hipSetDevice(device));
    if (g_device != device || !g_stream) {
        g_device = device;
        // default priority stream: prioritised streams are not used anywhere
        JAS_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    }
    return JAS_OK;
}

jas_stream_t jas_default_stream(void) { return (jas_stream_t)stream_or_default(nullptr); }

jas_status jas_malloc(void **p, size_t bytes)
{
    JAS_CHECK(p, JAS_ERR_INVALID, "jas_malloc: null out pointer");
    *p = nullptr;
    if (bytes == 0) return JAS_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(JAS_ERR_OOM, std::string("jas_malloc: ") + hipGetErrorString(e));
    }
    return JAS_OK;
}

jas_status jas_free(void *p)
{
    if (p) JAS_HIP(hipFree(p));
    return JAS_OK;
}

jas_status jas_memset(void *p, int v, size_t bytes, jas_stream_t s)
{
    if (bytes) JAS_HIP(hipMemsetAsync(p, v, bytes, stream_or_default(s)));
    return JAS_OK;
}

jas_status jas_memcpy_h2d(void *d, const void *h, size_t bytes, jas_stream_t s)
{
    if (bytes) {
        JAS_HIP(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, stream_or_default(s)));
        JAS_HIP(hipStreamSynchronize(stream_or_default(s)));  // h may be reused immediately
    }
    return JAS_OK;
}

jas_status jas_memcpy_d2h(void *h, const void *d, size_t bytes, jas_stream_t s)
{
    if (bytes) {
        JAS_HIP(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, stream_or_default(s)));
        JAS_HIP(hipStreamSynchronize(stream_or_default(s)));
    }
    return JAS_OK;
}

jas_status jas_memcpy_d2d(void *d, const void *src, size_t bytes, jas_stream_t s)
{
    if (bytes) JAS_HIP(hipMemcpyAsync(d, src, bytes, hipMemcpyDeviceToDevice, stream_or_default(s)));
    return JAS_OK;
}

jas_status jas_synchronize(jas_stream_t s)
{
    JAS_HIP(hipStreamSynchronize(stream_or_default(s)));
    return JAS_OK;
}

} // extern "C"
