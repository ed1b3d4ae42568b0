// Row reductions: softmax, LayerNorm, RMSNorm, and jasmine's generic
// sum/max/mean reductions.
//
// Reference: hsoftmax (mat_express_t.hpp:681-694) makes four materialised passes (hmax,
// exp, hsum, divide); layer_norm_net_t::forward (mat_net_t.hpp:209-225) five (vmean, sub,
// pow, vmean+sqrt, divide).  Here a row that fits the workgroup's registers is read from
// HBM once and written once: wave64 shuffles (DPP) reduce inside a wave, LDS across waves.
// Column-wise forms (jasmine's feature-major [d, T] LayerNorm normalises each column) map
// one thread per column so the loads stay coalesced across columns.
#include "jas_leaf.hpp"

#include <cfloat>

namespace jas {

typedef float floatx4 __attribute__((ext_vector_type(4)));

enum RowMode : int { RM_SOFTMAX = 0, RM_LN = 1, RM_RMS = 2 };

template <int NT, int PER, int MODE, bool V4>
__global__ void __launch_bounds__(NT)
rowop_reg_kernel(const float *__restrict__ x, float *__restrict__ y, int len, long vstride, long ystride, float eps,
                 const float *__restrict__ g, const float *__restrict__ bta)
{
    __shared__ float red[NT / WAVE];
    const float *xr = x + (long)blockIdx.x * vstride;
    float *yr = y + (long)blockIdx.x * ystride;
    const int t = threadIdx.x;
    float v[PER];
    if (V4) {
#pragma unroll
        for (int k = 0; k < PER / 4; ++k) {
            int e = (k * NT + t) * 4;
            // streaming input: non-temporal loads (the output is stored normally, below)
            floatx4 q = e < len ? __builtin_nontemporal_load((const floatx4 *)(xr + e)) : floatx4{0.f, 0.f, 0.f, 0.f};
            v[4 * k] = q[0]; v[4 * k + 1] = q[1]; v[4 * k + 2] = q[2]; v[4 * k + 3] = q[3];
        }
    } else {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            int e = k * NT + t;
            v[k] = e < len ? xr[e] : 0.f;
        }
    }
    auto idx = [&](int k) { return V4 ? ((k / 4) * NT + t) * 4 + (k % 4) : k * NT + t; };

    if (MODE == RM_SOFTMAX) {
        float m = -FLT_MAX;  // hmax starts from numeric_limits::lowest() (mat_express_t.hpp:619)
#pragma unroll
        for (int k = 0; k < PER; ++k)
            if (idx(k) < len && v[k] > m) m = v[k];
        m = block_max<NT>(m, red);
        // exp(x - m) = 2^(x log2(e) - m log2(e)): one fma and the hardware exp per element
        // (terms below 2^-126 flush to zero; the row max contributes 1), then one reciprocal
        // of the row sum for the whole row -- the VALU otherwise paid a full-precision expf and
        // an IEEE division per element
        const float l2e = 1.4426950408889634f, ml = m * l2e;
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            v[k] = idx(k) < len ? __builtin_amdgcn_exp2f(__builtin_fmaf(v[k], l2e, -ml)) : 0.f;
            s += v[k];
        }
        const float inv = 1.0f / block_sum<NT>(s, red);
#pragma unroll
        for (int k = 0; k < PER; ++k) v[k] *= inv;
    } else if (MODE == RM_LN) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < PER; ++k) s += v[k];  // padding is 0
        float mean = block_sum<NT>(s, red) / (float)len;
        float s2 = 0.f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            float d = idx(k) < len ? v[k] - mean : 0.f;
            s2 += d * d;
        }
        const float inv = 1.0f / sqrtf(block_sum<NT>(s2, red) / (float)len + eps);  // one per row
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            int e = idx(k) < len ? idx(k) : 0;
            v[k] = (v[k] - mean) * inv * (g ? g[e] : 1.f) + (bta ? bta[e] : 0.f);
        }
    } else {
        float s2 = 0.f;
#pragma unroll
        for (int k = 0; k < PER; ++k) s2 += v[k] * v[k];
        const float inv = 1.0f / sqrtf(block_sum<NT>(s2, red) / (float)len + eps);  // one per row
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            int e = idx(k) < len ? idx(k) : 0;
            v[k] = v[k] * inv * (g ? g[e] : 1.f);
        }
    }

    if (V4) {
#pragma unroll
        for (int k = 0; k < PER / 4; ++k) {
            int e = (k * NT + t) * 4;
            // an ordinary store: the output stays in the Infinity Cache for its consumer (a
            // nontemporal store streams it to HBM at once: 6.4 against 8.2 TB/s in a copy probe)
            if (e < len) *(floatx4 *)(yr + e) = floatx4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
        }
    } else {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            int e = k * NT + t;
            if (e < len) yr[e] = v[k];
        }
    }
}

// rows too long for registers: three passes over the row (later passes hit L2)
template <int NT, int MODE>
__global__ void __launch_bounds__(NT)
rowop_loop_kernel(const float *__restrict__ x, float *__restrict__ y, int len, long vstride, long ystride, float eps,
                  const float *__restrict__ g, const float *__restrict__ bta)
{
    __shared__ float red[NT / WAVE];
    const float *xr = x + (long)blockIdx.x * vstride;
    float *yr = y + (long)blockIdx.x * ystride;
    const int t = threadIdx.x;
    if (MODE == RM_SOFTMAX) {
        float m = -FLT_MAX;
        for (int e = t; e < len; e += NT) m = xr[e] > m ? xr[e] : m;
        m = block_max<NT>(m, red);
        float s = 0.f;
        const float l2e = 1.4426950408889634f, ml = m * l2e;  // exp as in rowop_reg_kernel
        for (int e = t; e < len; e += NT) s += __builtin_amdgcn_exp2f(__builtin_fmaf(xr[e], l2e, -ml));
        const float inv = 1.0f / block_sum<NT>(s, red);
        for (int e = t; e < len; e += NT) yr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(xr[e], l2e, -ml)) * inv;
    } else if (MODE == RM_LN) {
        float s = 0.f;
        for (int e = t; e < len; e += NT) s += xr[e];
        float mean = block_sum<NT>(s, red) / (float)len;
        float s2 = 0.f;
        for (int e = t; e < len; e += NT) { float d = xr[e] - mean; s2 += d * d; }
        const float inv = 1.0f / sqrtf(block_sum<NT>(s2, red) / (float)len + eps);
        for (int e = t; e < len; e += NT)
            yr[e] = (xr[e] - mean) * inv * (g ? g[e] : 1.f) + (bta ? bta[e] : 0.f);
    } else {
        float s2 = 0.f;
        for (int e = t; e < len; e += NT) s2 += xr[e] * xr[e];
        const float inv = 1.0f / sqrtf(block_sum<NT>(s2, red) / (float)len + eps);
        for (int e = t; e < len; e += NT) yr[e] = xr[e] * inv * (g ? g[e] : 1.f);
    }
}

// column form: a workgroup of 512 threads takes CW adjacent vectors (coalesced when they are
// adjacent columns of a row-major matrix, vstride == 1): lane l of the group serves vector
// l % CW, and the 512 / CW row groups split the elements, row group r taking elements
// r, r + RG, r + 2 RG, ...  Each thread accumulates its elements in order; the row groups'
// partials are combined in row-group order through LDS (deterministic for a given shape).
// With CACHE (len <= RG * 16) a thread keeps its elements in registers, so the vectors are
// read from memory once.
template <int MODE, int CW, bool CACHE>
__global__ void __launch_bounds__(512)
rowop_col_kernel(const float *__restrict__ x, float *__restrict__ y, int n_vec, int len, long vstride, long ystride,
                 long estride, float eps, const float *__restrict__ g, const float *__restrict__ bta)
{
#pragma clang fp contract(off)  // separate multiply and add, as jasmine's loops round them
    constexpr int RG = 512 / CW, PER = 16;
    __shared__ float red[RG][CW];
    const int c = threadIdx.x % CW, rg = threadIdx.x / CW;
    const int v = blockIdx.x * CW + c;
    const bool live = v < n_vec;
    const float *xr = x + (long)(live ? v : 0) * vstride;
    float *yr = y + (long)(live ? v : 0) * ystride;
    float xc[CACHE ? PER : 1];
    if (CACHE) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int e = rg + k * RG;
            xc[k] = (live && e < len) ? xr[e * estride] : 0.f;
        }
    }
    auto at = [&](int k, int e) { return CACHE ? xc[k] : xr[(long)e * estride]; };
    const int n_mine = live ? (len - rg + RG - 1) / RG : 0;  // elements of this thread
    auto combine = [&](float a, bool is_max) {
        red[rg][c] = a;
        __syncthreads();
        float t = red[0][c];
        for (int k = 1; k < RG; ++k) t = is_max ? fmaxf(t, red[k][c]) : t + red[k][c];
        __syncthreads();
        return t;
    };
#define JAS_COL_LOOP(BODY)                                                                                             \
    if (CACHE) {                                                                                                      \
        _Pragma("unroll") for (int k = 0; k < PER; ++k) if (k < n_mine) { const int e = rg + k * RG; BODY }           \
    } else {                                                                                                          \
        for (int k = 0; k < n_mine; ++k) { const int e = rg + k * RG; BODY }                                         \
    }
    if (MODE == RM_SOFTMAX) {
        float m = -FLT_MAX;
        JAS_COL_LOOP(m = fmaxf(m, at(k, e));)
        m = combine(m, true);
        float s = 0.f;
        const float l2e = 1.4426950408889634f, ml = m * l2e;  // exp as in rowop_reg_kernel
        JAS_COL_LOOP(s += __builtin_amdgcn_exp2f(__builtin_fmaf(at(k, e), l2e, -ml));)
        s = combine(s, false);
        const float inv = 1.0f / s;
        JAS_COL_LOOP(yr[(long)e * estride] = __builtin_amdgcn_exp2f(__builtin_fmaf(at(k, e), l2e, -ml)) * inv;)
    } else if (MODE == RM_LN) {
        float s = 0.f;
        JAS_COL_LOOP(s += at(k, e);)
        const float mean = combine(s, false) / (float)len;
        float s2 = 0.f;
        JAS_COL_LOOP(const float d = at(k, e) - mean; s2 += d * d;)
        const float inv = 1.0f / sqrtf(combine(s2, false) / (float)len + eps);
        JAS_COL_LOOP(yr[(long)e * estride] = (at(k, e) - mean) * inv * (g ? g[e] : 1.f) + (bta ? bta[e] : 0.f);)
    } else {
        float s2 = 0.f;
        JAS_COL_LOOP(s2 += at(k, e) * at(k, e);)
        const float inv = 1.0f / sqrtf(combine(s2, false) / (float)len + eps);
        JAS_COL_LOOP(yr[(long)e * estride] = at(k, e) * inv * (g ? g[e] : 1.f);)
    }
#undef JAS_COL_LOOP
}

// Column form on 16-byte column groups: adjacent vectors contiguous in memory (vstride ==
// ystride == 1), n_vec % 4 == 0, element stride a multiple of 4, 16-byte aligned.  Lane l of
// a row segment takes the four adjacent vectors 4 (l % L) .. +3 as one float4 (L = CW / 4
// lanes per row, so a wave's load covers 64 / L rows of 16 L bytes each -- four times the data
// per cache line touched of the one-float form); the 512 / L row groups split the elements as
// in rowop_col_kernel.  Each thread accumulates its elements in order; partials are combined
// over the lanes of a wave that serve the same vectors (butterfly over offsets L .. 32), then
// over the 8 waves in wave order (deterministic for a given shape).
template <int MODE, int CW, bool CACHE>
__global__ void __launch_bounds__(512)
rowop_col4_kernel(const float *__restrict__ x, float *__restrict__ y, int n_vec, int len, long estride, float eps,
                  const float *__restrict__ g, const float *__restrict__ bta)
{
#pragma clang fp contract(off)  // separate multiply and add, as jasmine's loops round them
    constexpr int L = CW / 4, RG = 512 / L, PER = 16;
    __shared__ floatx4 red[8][L];
    const int sg = threadIdx.x % L, rg = threadIdx.x / L, w = threadIdx.x / WAVE;
    const int v0 = blockIdx.x * CW + 4 * sg;
    const bool live = v0 < n_vec;
    const float *xr = x + (live ? v0 : 0);
    float *yr = y + (live ? v0 : 0);
    floatx4 xc[CACHE ? PER : 1];
    if (CACHE) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int e = rg + k * RG;
            xc[k] = (live && e < len) ? *(const floatx4 *)(xr + (long)e * estride) : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    auto at = [&](int k, int e) -> floatx4 { return CACHE ? xc[k] : *(const floatx4 *)(xr + (long)e * estride); };
    const int n_mine = live ? (len - rg + RG - 1) / RG : 0;
    auto combine = [&](floatx4 a, bool is_max) {
#pragma unroll
        for (int o = L; o < WAVE; o <<= 1) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float t = __shfl_xor(a[j], o, WAVE);
                a[j] = is_max ? fmaxf(a[j], t) : a[j] + t;
            }
        }
        if (threadIdx.x % WAVE < L) red[w][sg] = a;
        __syncthreads();
        floatx4 t = red[0][sg];
#pragma unroll
        for (int k = 1; k < 8; ++k) {
            const floatx4 r = red[k][sg];
#pragma unroll
            for (int j = 0; j < 4; ++j) t[j] = is_max ? fmaxf(t[j], r[j]) : t[j] + r[j];
        }
        __syncthreads();
        return t;
    };
#define JAS_COL4_LOOP(...)                                                                                            \
    if (CACHE) {                                                                                                      \
        _Pragma("unroll") for (int k = 0; k < PER; ++k) if (k < n_mine) { const int e = rg + k * RG; __VA_ARGS__ }           \
    } else {                                                                                                          \
        for (int k = 0; k < n_mine; ++k) { const int e = rg + k * RG; __VA_ARGS__ }                                         \
    }
    if (MODE == RM_SOFTMAX) {
        floatx4 m = {-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
        JAS_COL4_LOOP(const floatx4 a = at(k, e); for (int j = 0; j < 4; ++j) m[j] = fmaxf(m[j], a[j]);)
        m = combine(m, true);
        const float l2e = 1.4426950408889634f;
        floatx4 ml, s = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < 4; ++j) ml[j] = m[j] * l2e;
        JAS_COL4_LOOP(const floatx4 a = at(k, e);
                      for (int j = 0; j < 4; ++j) s[j] += __builtin_amdgcn_exp2f(__builtin_fmaf(a[j], l2e, -ml[j]));)
        s = combine(s, false);
        floatx4 inv;
        for (int j = 0; j < 4; ++j) inv[j] = 1.0f / s[j];
        JAS_COL4_LOOP(const floatx4 a = at(k, e); floatx4 o;
                      for (int j = 0; j < 4; ++j) o[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(a[j], l2e, -ml[j])) * inv[j];
                      *(floatx4 *)(yr + (long)e * estride) = o;)
    } else if (MODE == RM_LN) {
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
        JAS_COL4_LOOP(const floatx4 a = at(k, e); for (int j = 0; j < 4; ++j) s[j] += a[j];)
        s = combine(s, false);
        floatx4 mean, s2 = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < 4; ++j) mean[j] = s[j] / (float)len;
        JAS_COL4_LOOP(const floatx4 a = at(k, e); for (int j = 0; j < 4; ++j) { const float d = a[j] - mean[j]; s2[j] += d * d; })
        s2 = combine(s2, false);
        floatx4 inv;
        for (int j = 0; j < 4; ++j) inv[j] = 1.0f / sqrtf(s2[j] / (float)len + eps);
        JAS_COL4_LOOP(const floatx4 a = at(k, e); const float ge = g ? g[e] : 1.f, be = bta ? bta[e] : 0.f; floatx4 o;
                      for (int j = 0; j < 4; ++j) o[j] = (a[j] - mean[j]) * inv[j] * ge + be;
                      *(floatx4 *)(yr + (long)e * estride) = o;)
    } else {
        floatx4 s2 = {0.f, 0.f, 0.f, 0.f};
        JAS_COL4_LOOP(const floatx4 a = at(k, e); for (int j = 0; j < 4; ++j) s2[j] += a[j] * a[j];)
        s2 = combine(s2, false);
        floatx4 inv;
        for (int j = 0; j < 4; ++j) inv[j] = 1.0f / sqrtf(s2[j] / (float)len + eps);
        JAS_COL4_LOOP(const floatx4 a = at(k, e); const float ge = g ? g[e] : 1.f; floatx4 o;
                      for (int j = 0; j < 4; ++j) o[j] = a[j] * inv[j] * ge;
                      *(floatx4 *)(yr + (long)e * estride) = o;)
    }
#undef JAS_COL4_LOOP
}

template <int MODE, int CW>
static void launch_col4(const float *x, float *y, int n_vec, int len, long estride, float eps, const float *g,
                        const float *b, hipStream_t s)
{
    const dim3 grid(ceil_div(n_vec, CW));
    if (len <= (512 / (CW / 4)) * 16)
        hipLaunchKernelGGL((rowop_col4_kernel<MODE, CW, true>), grid, dim3(512), 0, s, x, y, n_vec, len, estride, eps, g, b);
    else
        hipLaunchKernelGGL((rowop_col4_kernel<MODE, CW, false>), grid, dim3(512), 0, s, x, y, n_vec, len, estride, eps, g, b);
}

template <int MODE, int CW>
static void launch_col(const float *x, float *y, int n_vec, int len, long vstride, long ystride, long estride,
                       float eps, const float *g, const float *b, hipStream_t s)
{
    const dim3 grid(ceil_div(n_vec, CW));
    if (len <= (512 / CW) * 16)
        hipLaunchKernelGGL((rowop_col_kernel<MODE, CW, true>), grid, dim3(512), 0, s, x, y, n_vec, len, vstride,
                           ystride, estride, eps, g, b);
    else
        hipLaunchKernelGGL((rowop_col_kernel<MODE, CW, false>), grid, dim3(512), 0, s, x, y, n_vec, len, vstride,
                           ystride, estride, eps, g, b);
}

template <int NT, int PER, int MODE>
static void launch_reg(const float *x, float *y, int n_vec, int len, long vstride, long ystride, float eps,
                       const float *g, const float *b, bool v4, hipStream_t s)
{
    if (v4)
        hipLaunchKernelGGL((rowop_reg_kernel<NT, PER, MODE, true>), dim3(n_vec), dim3(NT), 0, s, x, y, len, vstride,
                           ystride, eps, g, b);
    else
        hipLaunchKernelGGL((rowop_reg_kernel<NT, PER, MODE, false>), dim3(n_vec), dim3(NT), 0, s, x, y, len, vstride,
                           ystride, eps, g, b);
}

template <int MODE>
static jas_status rowop(const float *x, float *y, int n_vec, int len, long vstride, long ystride, long estride,
                        float eps, const float *g, const float *b, jas_stream_t stream)
{
    JAS_CHECK(x && y, JAS_ERR_INVALID, "row op: null pointer");
    JAS_CHECK(n_vec >= 0 && len > 0, JAS_ERR_INVALID, "row op: bad shape");
    if (n_vec == 0) return JAS_OK;
    JAS_CHECK(n_vec < (1 << 30), JAS_ERR_INVALID, "row op: too many vectors");
    hipStream_t s = stream_or_default(stream);
    if (estride != 1 && vstride == 1 && ystride == 1 && n_vec % 4 == 0 && estride % 4 == 0 &&
        (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0) {
        // adjacent columns of a row-major matrix in 16-byte groups: 8 vectors per workgroup
        // below 1024 of them, 16 from 1024 (jasmine's Transformer-base LayerNorm, [d, T]
        // with T = 512 / 1024: 7.1 -> 6.4 us and 13.1 -> 9.8 us per call against the
        // one-float form; 32 and 64 vectors per workgroup were slower: too few workgroups)
        if (n_vec >= 1024) launch_col4<MODE, 16>(x, y, n_vec, len, estride, eps, g, b, s);
        else launch_col4<MODE, 8>(x, y, n_vec, len, estride, eps, g, b, s);
        JAS_LAUNCH_CHECK();
        return JAS_OK;
    }
    if (estride != 1) {
        // the widest column group that still gives one workgroup per CU (64 columns: full
        // 256-byte rows per wave; 8: 32-byte segments, but 8x the workgroups)
        if ((long)ceil_div(n_vec, 64) >= 256) launch_col<MODE, 64>(x, y, n_vec, len, vstride, ystride, estride, eps, g, b, s);
        else if ((long)ceil_div(n_vec, 32) >= 256) launch_col<MODE, 32>(x, y, n_vec, len, vstride, ystride, estride, eps, g, b, s);
        else if ((long)ceil_div(n_vec, 16) >= 256) launch_col<MODE, 16>(x, y, n_vec, len, vstride, ystride, estride, eps, g, b, s);
        else launch_col<MODE, 8>(x, y, n_vec, len, vstride, ystride, estride, eps, g, b, s);
        JAS_LAUNCH_CHECK();
        return JAS_OK;
    }
    bool v4 = (len % 4 == 0) && (vstride % 4 == 0) && (ystride % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0);
    if (len <= 256) launch_reg<64, 4, MODE>(x, y, n_vec, len, vstride, ystride, eps, g, b, v4, s);
    else if (len <= 512) launch_reg<64, 8, MODE>(x, y, n_vec, len, vstride, ystride, eps, g, b, v4, s);
    else if (len <= 1024) launch_reg<128, 8, MODE>(x, y, n_vec, len, vstride, ystride, eps, g, b, v4, s);
    else if (len <= 2048) launch_reg<256, 8, MODE>(x, y, n_vec, len, vstride, ystride, eps, g, b, v4, s);
    else if (len <= 4096) launch_reg<256, 16, MODE>(x, y, n_vec, len, vstride, ystride, eps, g, b, v4, s);
    else if (len <= 8192) launch_reg<256, 32, MODE>(x, y, n_vec, len, vstride, ystride, eps, g, b, v4, s);
    else if (len <= 16384) launch_reg<512, 32, MODE>(x, y, n_vec, len, vstride, ystride, eps, g, b, v4, s);
    else hipLaunchKernelGGL((rowop_loop_kernel<512, MODE>), dim3(n_vec), dim3(512), 0, s, x, y, len, vstride, ystride, eps, g, b);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

// ---------------- whole-matrix softmax (mat_softmax_t, mat_express_t.hpp:642-659) ----------------
// pass 1: per block (max, sum exp(x - local max)); pass 2: one block combines; pass 3: write.
__global__ void __launch_bounds__(256) gsm_partial_kernel(const float *__restrict__ x, long n, float2 *part)
{
    __shared__ float red[4];
    float m = -FLT_MAX;
    long stride = (long)gridDim.x * 256;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) m = x[i] > m ? x[i] : m;
    m = block_max<256>(m, red);
    float s = 0.f;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) s += expf(x[i] - m);
    s = block_sum<256>(s, red);
    if (threadIdx.x == 0) part[blockIdx.x] = make_float2(m, s);
}

__global__ void __launch_bounds__(256) gsm_combine_kernel(float2 *part, int nb)
{
    __shared__ float red[4];
    float m = -FLT_MAX;
    for (int i = threadIdx.x; i < nb; i += 256) m = part[i].x > m ? part[i].x : m;
    m = block_max<256>(m, red);
    float s = 0.f;
    for (int i = threadIdx.x; i < nb; i += 256) s += part[i].y * expf(part[i].x - m);
    s = block_sum<256>(s, red);
    __syncthreads();
    if (threadIdx.x == 0) part[nb] = make_float2(m, s);
}

__global__ void __launch_bounds__(256) gsm_write_kernel(const float *__restrict__ x, float *y, long n, const float2 *ms)
{
    float2 r = *ms;
    long stride = (long)gridDim.x * 256;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) y[i] = expf(x[i] - r.x) / r.y;
}

// ---------------- generic reductions over a leaf (mat_express_t.hpp:511-628) ----------------
// Per-row and per-column forms use one thread per output and accumulate sequentially in
// the output type, exactly the order jasmine's loops use (hsum :548-564, vsum :530-546).
template <typename T>
__device__ __forceinline__ T leaf_get(const LeafDev &L, int i, int j)
{
    return (T)load_elem(L.p, leaf_index(L, i, j), L.dtype);
}

template <typename T>
__global__ void reduce_line_kernel(LeafDev L, int rows, int cols, int op, int axis, T *out)
{
    int o = blockIdx.x * blockDim.x + threadIdx.x;
    int n_out = axis == 0 ? rows : cols;
    if (o >= n_out) return;
    int len = axis == 0 ? cols : rows;
    T acc = op == 1 ? -std::numeric_limits<T>::max() : (T)0;
    for (int k = 0; k < len; ++k) {
        T v = axis == 0 ? leaf_get<T>(L, o, k) : leaf_get<T>(L, k, o);
        if (op == 1) acc = v > acc ? v : acc;
        else acc += v;
    }
    if (op == 2) acc = acc / (T)len;  // vmean / hmean: ele / int (mat_express_t.hpp:566-578)
    out[o] = acc;
}

// whole-matrix: per-row sequential partials, then a sequential pass over the partials
template <typename T>
__global__ void reduce_all_kernel(const T *rowpart, int rows, int cols, int op, T *out)
{
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    T acc = op == 1 ? -std::numeric_limits<T>::max() : (T)0;
    for (int r = 0; r < rows; ++r) {
        if (op == 1) acc = rowpart[r] > acc ? rowpart[r] : acc;
        else acc += rowpart[r];
    }
    if (op == 2) acc = acc / (T)((long)rows * cols);  // mean (mat_express_t.hpp:580-585)
    out[0] = acc;
}

template <typename T>
static jas_status reduce_t(const jas_leaf *in, int op, int axis, void *d_out, hipStream_t s)
{
    int rows = in->vrows, cols = in->vcols;
    LeafDev L = classify(*in, rows, cols);
    if (L.kind == LK_CONTIG) {  // contiguous row-major: strided form of the same address
        L.kind = LK_STRIDED;
        L.rs = cols;
        L.cs = 1;
    }
    if (axis == 0 || axis == 1) {
        int n_out = axis == 0 ? rows : cols;
        hipLaunchKernelGGL(reduce_line_kernel<T>, dim3(ceil_div(n_out, 128)), dim3(128), 0, s, L, rows, cols, op,
                           axis, (T *)d_out);
        JAS_LAUNCH_CHECK();
        return JAS_OK;
    }
    T *part = (T *)workspace(sizeof(T) * (size_t)rows, s);
    JAS_CHECK(part, JAS_ERR_OOM, "jas_reduce: workspace allocation failed");
    hipLaunchKernelGGL(reduce_line_kernel<T>, dim3(ceil_div(rows, 128)), dim3(128), 0, s, L, rows, cols,
                       op == 2 ? 0 : op, 0, part);
    hipLaunchKernelGGL(reduce_all_kernel<T>, dim3(1), dim3(64), 0, s, part, rows, cols, op, (T *)d_out);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

// ---------------- residual update + norm (decode) ----------------
// x[n] += (sum_s part[s][n] + bias); y[n] = norm(x[n]) * g (+ b).  `part` holds the K-split
// partial sums of the projection that feeds the residual stream ([split][16][d], split
// order), so the split-K reduction costs no launch of its own.  One workgroup per token.
constexpr int RN_MAX_SPLITS = 8;  // the decode projections split K at most 8 ways
template <int PER, bool RMS, int NT>
__global__ void __launch_bounds__(NT)
resid_norm_kernel(float *__restrict__ x, const float *__restrict__ part, int ks, const float *__restrict__ bias,
                  const float *__restrict__ g, const float *__restrict__ bta, float *__restrict__ y, int d, float eps,
                  int y_packed)
{
    __shared__ float red[NT / 64];
    const int n = blockIdx.x, t = threadIdx.x;
    float *xr = x + (long)n * d;
    float v[PER];
    // the norm's gain (and bias) are requested together with the row, not after the
    // reductions: one memory round trip fewer on the critical path
    float4 gg[PER / 4], bb4[PER / 4];
#pragma unroll
    for (int k = 0; k < PER / 4; ++k) {
        const int e = (k * NT + t) * 4;
        gg[k] = e < d ? *(const float4 *)(g + e) : make_float4(0.f, 0.f, 0.f, 0.f);
        bb4[k] = (!RMS && bta && e < d) ? *(const float4 *)(bta + e) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < PER / 4; ++k) {
        const int e = (k * NT + t) * 4;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        if (e < d) {
            a = *(const float4 *)(xr + e);
            if (ks > 0) {
                // every split's partial is requested before the first is added (one round
                // trip, not ks); the sum keeps split order
                float4 q[RN_MAX_SPLITS];
#pragma unroll
                for (int sp = 0; sp < RN_MAX_SPLITS; ++sp)
                    if (sp < ks) q[sp] = *(const float4 *)(part + ((long)sp * 16 + n) * d + e);
                float4 sacc = q[0];
#pragma unroll
                for (int sp = 1; sp < RN_MAX_SPLITS; ++sp)
                    if (sp < ks) { sacc.x += q[sp].x; sacc.y += q[sp].y; sacc.z += q[sp].z; sacc.w += q[sp].w; }
                if (bias) {
                    float4 bb = *(const float4 *)(bias + e);
                    sacc.x += bb.x; sacc.y += bb.y; sacc.z += bb.z; sacc.w += bb.w;
                }
                a.x += sacc.x; a.y += sacc.y; a.z += sacc.z; a.w += sacc.w;
                *(float4 *)(xr + e) = a;
            }
        }
        v[4 * k] = a.x; v[4 * k + 1] = a.y; v[4 * k + 2] = a.z; v[4 * k + 3] = a.w;
    }
    float mean = 0.f;
    if (!RMS) {
        float sm = 0.f;
#pragma unroll
        for (int k = 0; k < PER; ++k) sm += v[k];
        mean = block_sum<NT>(sm, red) / (float)d;
    }
    float s2 = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int e = ((k / 4) * NT + t) * 4;
        const float dv = e < d ? v[k] - mean : 0.f;
        s2 += dv * dv;
    }
    const float inv = 1.0f / sqrtf(block_sum<NT>(s2, red) / (float)d + eps);  // one reciprocal per token
#pragma unroll
    for (int k = 0; k < PER / 4; ++k) {
        const int e = (k * NT + t) * 4;
        if (e >= d) continue;
        float4 o;
        o.x = (v[4 * k] - mean) * inv * gg[k].x;
        o.y = (v[4 * k + 1] - mean) * inv * gg[k].y;
        o.z = (v[4 * k + 2] - mean) * inv * gg[k].z;
        o.w = (v[4 * k + 3] - mean) * inv * gg[k].w;
        if (!RMS && bta) {
            o.x += bb4[k].x; o.y += bb4[k].y; o.z += bb4[k].z; o.w += bb4[k].w;
        }
        // packed: the 4 features e..e+3 of token n are one lane's B-operand float4
        const long yo = y_packed ? ((long)(e >> 4) * 64 + n + 16 * ((e & 15) >> 2)) * 4 : (long)n * d + e;
        *(float4 *)(y + yo) = o;
    }
}

jas_status resid_norm(float *x, const float *part, int ks, const float *bias, const float *g, const float *b, float *y,
                      int N, int d, float eps, bool rms, hipStream_t s, bool y_packed)
{
    JAS_CHECK(d % 4 == 0 && d <= 8192 && N >= 1 && N <= 16 && g, JAS_ERR_INVALID, "resid_norm: unsupported shape");
    JAS_CHECK(ks <= RN_MAX_SPLITS, JAS_ERR_INVALID, "resid_norm: more K splits than supported");
    JAS_CHECK(!y_packed || d % 16 == 0, JAS_ERR_INVALID, "resid_norm: packed output needs d % 16 == 0");
    const int yp = y_packed ? 1 : 0;
#define JAS_RN(PER, NT)                                                                                      \
    if (d <= PER * NT) {                                                                                     \
        if (rms) hipLaunchKernelGGL((resid_norm_kernel<PER, true, NT>), dim3(N), dim3(NT), 0, s, x, part, ks, \
                                    bias, g, b, y, d, eps, yp);                                              \
        else hipLaunchKernelGGL((resid_norm_kernel<PER, false, NT>), dim3(N), dim3(NT), 0, s, x, part, ks,   \
                                bias, g, b, y, d, eps, yp);                                                  \
        JAS_LAUNCH_CHECK();                                                                                  \
        return JAS_OK;                                                                                       \
    }
    // one float4 per thread up to d = 4096 (more waves per token: the partial loads are
    // spread over 16 waves instead of 4); wider rows take 8 features per thread
    JAS_RN(4, 256) JAS_RN(4, 512) JAS_RN(4, 1024) JAS_RN(8, 1024)
#undef JAS_RN
    return fail(JAS_ERR_INVALID, "resid_norm: d too large");
}

template <typename T>
__global__ void causal_mask_kernel(T *S, int rows, int cols, long ld, T value)
{
    long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (long)rows * cols) return;
    int i = (int)(g / cols), j = (int)(g % cols);
    if (j > i) S[(long)i * ld + j] = value;
}

} // namespace jas

using namespace jas;

extern "C" {

jas_status jas_causal_mask(float *S, int rows, int cols, long ld, float value, jas_stream_t stream)
{
    JAS_CHECK(S && rows >= 0 && cols >= 0 && ld >= cols, JAS_ERR_INVALID, "jas_causal_mask: bad arguments");
    long n = (long)rows * cols;
    if (n) hipLaunchKernelGGL(causal_mask_kernel<float>, dim3(ceil_div(n, 256)), dim3(256), 0, stream_or_default(stream),
                              S, rows, cols, ld, value);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

jas_status jas_causal_mask_f64(double *S, int rows, int cols, long ld, double value, jas_stream_t stream)
{
    JAS_CHECK(S && rows >= 0 && cols >= 0 && ld >= cols, JAS_ERR_INVALID, "jas_causal_mask: bad arguments");
    long n = (long)rows * cols;
    if (n) hipLaunchKernelGGL(causal_mask_kernel<double>, dim3(ceil_div(n, 256)), dim3(256), 0,
                              stream_or_default(stream), S, rows, cols, ld, value);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

jas_status jas_softmax(const float *x, float *y, int n_vec, int len, long vstride, long ystride, long estride,
                       jas_stream_t s)
{
    return rowop<RM_SOFTMAX>(x, y, n_vec, len, vstride, ystride, estride, 0.f, nullptr, nullptr, s);
}

jas_status jas_layernorm(const float *x, float *y, int n_vec, int len, long vstride, long ystride, long estride,
                         float eps, const float *g, const float *b, jas_stream_t s)
{
    return rowop<RM_LN>(x, y, n_vec, len, vstride, ystride, estride, eps, g, b, s);
}

jas_status jas_rmsnorm(const float *x, float *y, int n_vec, int len, long vstride, long ystride, long estride,
                       float eps, const float *g, jas_stream_t s)
{
    return rowop<RM_RMS>(x, y, n_vec, len, vstride, ystride, estride, eps, g, nullptr, s);
}

jas_status jas_softmax_global(const float *x, float *y, long n, jas_stream_t stream)
{
    JAS_CHECK(x && y && n > 0, JAS_ERR_INVALID, "jas_softmax_global: bad arguments");
    hipStream_t s = stream_or_default(stream);
    int nb = (int)std::min<long>(1024, (n + 255) / 256);
    float2 *part = (float2 *)workspace(sizeof(float2) * (nb + 1), s);
    JAS_CHECK(part, JAS_ERR_OOM, "jas_softmax_global: workspace allocation failed");
    hipLaunchKernelGGL(gsm_partial_kernel, dim3(nb), dim3(256), 0, s, x, n, part);
    hipLaunchKernelGGL(gsm_combine_kernel, dim3(1), dim3(256), 0, s, part, nb);
    hipLaunchKernelGGL(gsm_write_kernel, dim3(nb), dim3(256), 0, s, x, y, n, (const float2 *)(part + nb));
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

jas_status jas_reduce(const jas_leaf *in, int op, int axis, void *d_out, int32_t out_dtype, jas_stream_t stream)
{
    JAS_CHECK(in && d_out, JAS_ERR_INVALID, "jas_reduce: null argument");
    JAS_CHECK(op >= 0 && op <= 2 && axis >= 0 && axis <= 2, JAS_ERR_INVALID, "jas_reduce: bad op/axis");
    JAS_CHECK(in->vrows > 0 && in->vcols > 0 && in->rows > 0 && in->cols > 0, JAS_ERR_INVALID,
              "jas_reduce: empty input");
    hipStream_t s = stream_or_default(stream);
    if (out_dtype == JAS_F64) return reduce_t<double>(in, op, axis, d_out, s);
    JAS_CHECK(out_dtype == JAS_F32, JAS_ERR_INVALID, "jas_reduce: out dtype must be f32 or f64");
    return reduce_t<float>(in, op, axis, d_out, s);
}

} // extern "C"
