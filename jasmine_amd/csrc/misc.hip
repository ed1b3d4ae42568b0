// Rotary embeddings, token embedding gather, argmax, seeded normal fill.
#include "jas_common.hpp"

#include <cfloat>

namespace jas {

// mat_RoPE_t::init cache entry (mat_RoPE_t.hpp:107-131) for val_type float:
// angle = (float)(c / pow(10000.0, (float)(r/2) / (float)d)); cos where r, c have equal
// parity, -sin at (even, odd), sin at (odd, even).
template <typename T>
__device__ __forceinline__ T rope_jas_entry(int r, int c, int d)
{
    // (i / 2) / static_cast<val_type>(m_d) and the angle are val_type; pow is double
    T e = (T)(r / 2) / (T)d;
    T angle = (T)((double)c / pow(10000.0, (double)e));
    if ((r & 1) == (c & 1)) return cos(angle);
    return (r & 1) ? sin(angle) : -sin(angle);
}

// RoPE_net_t::forward (mat_RoPE_t.hpp:166-188): y[2i+r, m] = sum_c block(r, c) x[2i+c, m],
// a float dot of two terms accumulated from 0 (no fused multiply-add).
template <typename V>
__global__ void rope_jas_kernel(const V *__restrict__ x, V *__restrict__ y, int d, int T)
{
#pragma clang fp contract(off)
    long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    int half = d / 2;
    if (g >= (long)half * T) return;
    int i = (int)(g / T), m = (int)(g % T);
    V x0 = x[(long)(2 * i) * T + m], x1 = x[(long)(2 * i + 1) * T + m];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        V s = (V)0;
        s = s + rope_jas_entry<V>(2 * i + r, 2 * m, d) * x0;
        s = s + rope_jas_entry<V>(2 * i + r, 2 * m + 1, d) * x1;
        y[(long)(2 * i + r) * T + m] = s;
    }
}

template <typename V>
__global__ void zero_row_kernel(V *y, int T)
{
    int m = blockIdx.x * blockDim.x + threadIdx.x;
    if (m < T) y[m] = (V)0;
}

template <typename V>
static jas_status rope_jas(const V *x, V *y, int d, int T, jas_stream_t stream)
{
    JAS_CHECK(x && y && d > 0 && T > 0, JAS_ERR_INVALID, "jas_rope_jasmine: bad arguments");
    hipStream_t s = stream_or_default(stream);
    long n = (long)(d / 2) * T;
    if (n) hipLaunchKernelGGL(rope_jas_kernel<V>, dim3(ceil_div(n, 256)), dim3(256), 0, s, x, y, d, T);
    if (d & 1)  // the odd trailing row of the zero-initialised result stays 0 (mat_RoPE_t.hpp:176-186)
        hipLaunchKernelGGL(zero_row_kernel<V>, dim3(ceil_div(T, 256)), dim3(256), 0, s, y + (long)(d - 1) * T, T);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

// LLaMA rotary, interleaved pairs, angles in double (positions reach thousands of radians)
__global__ void rope_llama_kernel(float *x, const int32_t *__restrict__ pos, int n, int nh, int dh, long tstride,
                                  float theta)
{
    long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    int hp = dh / 2;
    long total = (long)n * nh * hp;
    if (g >= total) return;
    int i = (int)(g % hp);
    long r = g / hp;
    int h = (int)(r % nh);
    int t = (int)(r / nh);
    double inv = pow((double)theta, -2.0 * i / (double)dh);
    double a = (double)pos[t] * inv;
    double c = cos(a), s = sin(a);
    float *p = x + (long)t * tstride + (long)h * dh + 2 * i;
    double x0 = p[0], x1 = p[1];
    p[0] = (float)(x0 * c - x1 * s);
    p[1] = (float)(x0 * s + x1 * c);
}

__global__ void embed_kernel(const float *__restrict__ wte, const float *__restrict__ wpe, const int32_t *__restrict__ ids,
                             const int32_t *__restrict__ pos, float *__restrict__ out, int n, int d)
{
    long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (long)n * d) return;
    int t = (int)(g / d), e = (int)(g % d);
    float v = wte[(long)ids[t] * d + e];
    if (wpe) v = v + wpe[(long)pos[t] * d + e];
    out[g] = v;
}

// argmax of each row; ties go to the lowest index (the first maximum, like a forward scan).
// Two passes: chunks of ARGMAX_CHUNK elements of every row are scanned by their own
// workgroups (a 50257-long row is 13 of them, so the scan is not one workgroup's latency
// chain), then one workgroup per row reduces the chunk winners.
constexpr int ARGMAX_CHUNK = 4096;

__device__ __forceinline__ void argmax_combine(float &bv, int &bi, float ov, int oi)
{
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// block-wide (256 threads) first-maximum reduction; thread 0 gets the result
__device__ __forceinline__ void argmax_block(float &bv, int &bi)
{
    __shared__ float sv[4];
    __shared__ int si[4];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_combine(bv, bi, __shfl_xor(bv, o, WAVE), __shfl_xor(bi, o, WAVE));
    const int w = threadIdx.x / WAVE;
    if (threadIdx.x % WAVE == 0) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int k = 1; k < 4; ++k) argmax_combine(bv, bi, sv[k], si[k]);
}

__global__ void __launch_bounds__(256) argmax_chunk_kernel(const float *__restrict__ x, int V, long ld,
                                                           float *__restrict__ pv, int *__restrict__ pi)
{
    const int row = blockIdx.y, c = blockIdx.x, nch = gridDim.x;
    const float *r = x + (long)row * ld;
    const int e0 = c * ARGMAX_CHUNK, e1 = min(V, e0 + ARGMAX_CHUNK);
    float v[ARGMAX_CHUNK / 256];
#pragma unroll
    for (int k = 0; k < ARGMAX_CHUNK / 256; ++k) {  // all loads in flight before the scan
        const int e = e0 + k * 256 + threadIdx.x;
        v[k] = e < e1 ? r[e] : -INFINITY;
    }
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < ARGMAX_CHUNK / 256; ++k) {
        const int e = e0 + k * 256 + threadIdx.x;
        if (e < e1 && v[k] > bv) { bv = v[k]; bi = e; }
    }
    argmax_block(bv, bi);
    if (threadIdx.x == 0) {
        pv[(long)row * nch + c] = bv;
        pi[(long)row * nch + c] = bi;
    }
}

__global__ void __launch_bounds__(256) argmax_final_kernel(const float *__restrict__ pv, const int *__restrict__ pi,
                                                           int nch, int32_t *out)
{
    const int row = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int c = threadIdx.x; c < nch; c += 256) argmax_combine(bv, bi, pv[(long)row * nch + c], pi[(long)row * nch + c]);
    argmax_block(bv, bi);
    if (threadIdx.x == 0) out[row] = bi == 0x7fffffff ? 0 : bi;
}

size_t argmax_workspace_bytes(int n, int V)
{
    return (size_t)n * ((V + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK) * (sizeof(float) + sizeof(int));
}

jas_status argmax_impl(const float *x, int n, int V, long ld, int32_t *out, void *work, hipStream_t s)
{
    if (!n) return JAS_OK;
    const int nch = (V + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    float *pv = (float *)work;
    int *pi = (int *)(pv + (size_t)n * nch);
    hipLaunchKernelGGL(argmax_chunk_kernel, dim3(nch, n), dim3(256), 0, s, x, V, ld, pv, pi);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(n), dim3(256), 0, s, pv, pi, nch, out);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

__global__ void fill_normal_kernel(float *x, size_t n, uint64_t key, float mean, float std)
{
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t a = splitmix64(key + 2 * i), b = splitmix64(key + 2 * i + 1);
        double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        x[i] = (float)((double)mean + (double)std * z);
    }
}

} // namespace jas

using namespace jas;

// Achievable streaming-read rate (bandwidth calibration, not a jasmine operation): every
// thread reads 16-byte chunks grid-stride, U loads in flight, and folds them into one word
// that is stored only if it equals a value no input makes likely, so the reads cannot be
// removed.  NT: nontemporal loads, as the decode kernels issue them.
template <int U, bool NT>
__global__ void __launch_bounds__(256) read_probe_kernel(const u32x4 *__restrict__ a, long n16, unsigned *sink)
{
    const long stride = (long)gridDim.x * 256;
    unsigned acc = 0;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long j = min(i + u * stride, n16 - 1);
            v[u] = NT ? __builtin_nontemporal_load(a + j) : a[j];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

extern "C" {

jas_status jas_rope_jasmine(const float *x, float *y, int d, int T, jas_stream_t stream)
{
    return rope_jas<float>(x, y, d, T, stream);
}

jas_status jas_rope_jasmine_f64(const double *x, double *y, int d, int T, jas_stream_t stream)
{
    return rope_jas<double>(x, y, d, T, stream);
}

jas_status jas_rope_llama(float *x, const int32_t *pos, int n, int nh, int dh, long tstride, float theta,
                          jas_stream_t stream)
{
    JAS_CHECK(x && pos && n >= 0 && nh > 0 && dh > 0 && dh % 2 == 0, JAS_ERR_INVALID, "jas_rope_llama: bad arguments");
    long total = (long)n * nh * (dh / 2);
    if (total)
        hipLaunchKernelGGL(rope_llama_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, stream_or_default(stream), x,
                           pos, n, nh, dh, tstride, theta);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

jas_status jas_embed(const float *wte, const float *wpe, const int32_t *ids, const int32_t *pos, float *out, int n,
                     int d, jas_stream_t stream)
{
    JAS_CHECK(wte && ids && out && n >= 0 && d > 0 && (!wpe || pos), JAS_ERR_INVALID, "jas_embed: bad arguments");
    long total = (long)n * d;
    if (total)
        hipLaunchKernelGGL(embed_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, stream_or_default(stream), wte, wpe,
                           ids, pos, out, n, d);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

jas_status jas_argmax(const float *x, int n, int V, long ld, int32_t *out, jas_stream_t stream)
{
    JAS_CHECK(x && out && n >= 0 && V > 0 && ld >= V, JAS_ERR_INVALID, "jas_argmax: bad arguments");
    if (!n) return JAS_OK;
    JAS_CHECK(n <= 65535, JAS_ERR_INVALID, "jas_argmax: at most 65535 rows");
    hipStream_t s = stream_or_default(stream);
    void *work = workspace(argmax_workspace_bytes(n, V), s);
    JAS_CHECK(work, JAS_ERR_OOM, "jas_argmax: workspace allocation failed");
    return argmax_impl(x, n, V, ld, out, work, s);
}

jas_status jas_fill_normal(float *x, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std,
                           jas_stream_t stream)
{
    JAS_CHECK(x || n == 0, JAS_ERR_INVALID, "jas_fill_normal: null pointer");
    if (!n) return JAS_OK;
    unsigned nb = (unsigned)std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(fill_normal_kernel, dim3(nb), dim3(256), 0, stream_or_default(stream), x, n,
                       stream_key(seed, stream_id), mean, std);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

jas_status jas_hbm_read_probe(const void *d_buf, size_t bytes, int workgroups, int loads_in_flight, int nontemporal,
                              unsigned *d_sink, jas_stream_t stream)
{
    JAS_CHECK(d_buf && d_sink && bytes >= 16 && bytes % 16 == 0 && (uintptr_t)d_buf % 16 == 0, JAS_ERR_INVALID,
              "jas_hbm_read_probe: need a 16-byte aligned buffer of a multiple of 16 bytes");
    JAS_CHECK(workgroups > 0 && (loads_in_flight == 4 || loads_in_flight == 8), JAS_ERR_INVALID,
              "jas_hbm_read_probe: workgroups > 0, 4 or 8 loads in flight");
    const long n16 = (long)(bytes / 16);
    hipStream_t s = stream_or_default(stream);
    const u32x4 *a = (const u32x4 *)d_buf;
    if (loads_in_flight == 4 && nontemporal) hipLaunchKernelGGL((read_probe_kernel<4, true>), dim3(workgroups), dim3(256), 0, s, a, n16, d_sink);
    else if (loads_in_flight == 4) hipLaunchKernelGGL((read_probe_kernel<4, false>), dim3(workgroups), dim3(256), 0, s, a, n16, d_sink);
    else if (nontemporal) hipLaunchKernelGGL((read_probe_kernel<8, true>), dim3(workgroups), dim3(256), 0, s, a, n16, d_sink);
    else hipLaunchKernelGGL((read_probe_kernel<8, false>), dim3(workgroups), dim3(256), 0, s, a, n16, d_sink);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

} // extern "C"
