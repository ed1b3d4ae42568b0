// Runtime part of the C ABI: device selection, library stream, memory, errors, RNG fill.
// Storage behind jasmine's mat_t (mat_t.hpp:53-69 allocate+zero, :30-42 release).
#include "jas_common.hpp"

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <vector>

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

// Library-internal scratch for multi-pass kernels (partials of whole-matrix reductions,
// prefill key-split partials, argmax partials): one buffer per stream, so work queued on
// different streams never shares partials.  Calls on one stream run in order, so reuse
// between them is safe; a buffer grows only after its own stream has drained (the old
// buffer may still be read by queued kernels).  Issuing calls on one stream from two host
// threads at once is not supported (neither is it by the reference, which has no threads).
// A buffer lives until jas_stream_release_scratch(stream) or the process ends.
struct Scratch {
    void *p = nullptr;
    size_t bytes = 0;
};
static std::mutex g_ws_mu;
static std::unordered_map<hipStream_t, Scratch> g_ws;
void *workspace(size_t bytes, hipStream_t s)
{
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Scratch &w = g_ws[s];
    if (bytes <= w.bytes) return w.p;
    if (w.p) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(w.p);
    }
    size_t nb = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (hipMalloc(&w.p, nb) != hipSuccess) {
        w.p = nullptr;
        w.bytes = 0;
        return nullptr;
    }
    w.bytes = nb;
    return w.p;
}

// Split-arrival counters (decode attention's in-kernel merge), one zeroed array per stream.
// Kernels leave every counter at zero, so an array is zeroed only when it is allocated; it
// grows (after its stream has drained) like the scratch above.
static std::unordered_map<hipStream_t, Scratch> g_ctr;
unsigned *arrival_counters(size_t n, hipStream_t s)
{
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Scratch &w = g_ctr[s];
    const size_t bytes = n * sizeof(unsigned);
    if (bytes <= w.bytes) return (unsigned *)w.p;
    if (w.p) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(w.p);
    }
    const size_t nb = bytes < 4096 ? 4096 : bytes;
    w.p = nullptr;
    w.bytes = 0;
    if (hipMalloc(&w.p, nb) != hipSuccess) return (unsigned *)(w.p = nullptr);
    if (hipMemset(w.p, 0, nb) != hipSuccess) {  // synchronous: never part of a captured graph
        (void)hipFree(w.p);
        w.p = nullptr;
        return nullptr;
    }
    w.bytes = nb;
    return (unsigned *)w.p;
}

jas_status release_workspace(hipStream_t s)
{
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto it = g_ws.find(s);
    auto ic = g_ctr.find(s);
    if (it == g_ws.end() && ic == g_ctr.end()) return JAS_OK;
    JAS_HIP(hipStreamSynchronize(s));  // queued kernels may still read the buffers
    if (it != g_ws.end()) {
        if (it->second.p) JAS_HIP(hipFree(it->second.p));
        g_ws.erase(it);
    }
    if (ic != g_ctr.end()) {
        if (ic->second.p) JAS_HIP(hipFree(ic->second.p));
        g_ctr.erase(ic);
    }
    return JAS_OK;
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

jas_status jas_stream_release_scratch(jas_stream_t stream)
{
    return release_workspace(stream_or_default(stream));
}

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

} // extern "C"

namespace jas {
namespace {
// Stream-ordered cache of device blocks behind the C++ headers' matrices.  Every device
// operation the headers issue runs on the library stream, so a block released by the host
// may be handed to the next allocation at once: work that uses it later is queued behind
// the work that used it before.  Sizes are rounded to 1/8 of their power of two (at least
// 512 bytes), blocks are reused by rounded size, and the cache is emptied (after a stream
// synchronisation) when it holds more than kMaxCached or an allocation fails.
struct Pool {
    std::mutex mu;
    std::unordered_map<size_t, std::vector<void *>> free_by_size;
    std::unordered_map<void *, size_t> live;
    size_t cached = 0;
    static constexpr size_t kMaxCached = 16ull << 30;
};
Pool &pool()
{
    static Pool *p = new Pool;  // never destroyed: no device call after the runtime's teardown
    return *p;
}
size_t pool_round(size_t b)
{
    if (b <= 512) return 512;
    size_t p2 = 1;
    while (p2 < b) p2 <<= 1;
    const size_t g = std::max<size_t>(512, p2 / 8);
    return (b + g - 1) / g * g;
}
// caller holds the lock
hipError_t pool_drain(Pool &pl)
{
    hipError_t e = hipSuccess;
    if (!pl.cached) return e;
    if (g_stream) e = hipStreamSynchronize(g_stream);
    for (auto &kv : pl.free_by_size)
        for (void *q : kv.second) {
            const hipError_t f = hipFree(q);
            if (e == hipSuccess) e = f;
        }
    pl.free_by_size.clear();
    pl.cached = 0;
    return e;
}
} // namespace
} // namespace jas

extern "C" {

jas_status jas_pool_alloc(void **p, size_t bytes)
{
    JAS_CHECK(p, JAS_ERR_INVALID, "jas_pool_alloc: null out pointer");
    *p = nullptr;
    const size_t r = pool_round(bytes ? bytes : 1);
    Pool &pl = pool();
    std::lock_guard<std::mutex> lk(pl.mu);
    auto it = pl.free_by_size.find(r);
    if (it != pl.free_by_size.end() && !it->second.empty()) {
        *p = it->second.back();
        it->second.pop_back();
        pl.cached -= r;
    } else {
        hipError_t e = hipMalloc(p, r);
        if (e != hipSuccess) {  // give the cached blocks back and try once more
            (void)hipGetLastError();
            (void)pool_drain(pl);
            e = hipMalloc(p, r);
        }
        if (e != hipSuccess) {
            *p = nullptr;
            return fail(JAS_ERR_OOM, std::string("jas_pool_alloc: ") + hipGetErrorString(e));
        }
    }
    pl.live[*p] = r;
    return JAS_OK;
}

jas_status jas_pool_free(void *p)
{
    if (!p) return JAS_OK;
    Pool &pl = pool();
    std::lock_guard<std::mutex> lk(pl.mu);
    auto it = pl.live.find(p);
    JAS_CHECK(it != pl.live.end(), JAS_ERR_INVALID, "jas_pool_free: not a pool block");
    const size_t r = it->second;
    pl.live.erase(it);
    pl.free_by_size[r].push_back(p);
    pl.cached += r;
    if (pl.cached > Pool::kMaxCached) JAS_HIP(pool_drain(pl));
    return JAS_OK;
}

jas_status jas_pool_trim(size_t *cached_before)
{
    Pool &pl = pool();
    std::lock_guard<std::mutex> lk(pl.mu);
    if (cached_before) *cached_before = pl.cached;
    JAS_HIP(pool_drain(pl));
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
