// Shared helpers for the gfx950 kernels and the C ABI implementation.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstring>
#include <cstdio>
#include <string>

#include "../../include/jasmine_hip.h"

namespace jas {

// thread-local last error message behind jas_last_error()
void set_error(const std::string &msg);
jas_status fail(jas_status code, const std::string &msg);
hipStream_t stream_or_default(jas_stream_t s);
void *workspace(size_t bytes, hipStream_t s);
// n zeroed split-arrival counters for kernels on stream s (one array per stream, left zero
// by every kernel that uses it); nullptr when out of memory
unsigned *arrival_counters(size_t n, hipStream_t s);
// frees the stream's scratch and counters after its queued work has drained
jas_status release_workspace(hipStream_t s);
// x[n] += sum_s part[(s*16 + n)*d ...] + bias; y = norm(x) (RMSNorm, or LayerNorm with b)
jas_status resid_norm(float *x, const float *part, int ks, const float *bias, const float *g, const float *b, float *y,
                      int N, int d, float eps, bool rms, hipStream_t s, bool y_packed = false);
// decode attention with an optional packed-B output (o_packed_d = H*D features) for the
// next packed GEMM; 0 = the jas_attn_decode layout O[b][h][D]
// kv_bf16: K/V hold bf16 elements (same element strides)
jas_status attn_decode_impl(const float *q, const void *K, const void *V, float *O, const int32_t *seqlens, int B,
                            int H, int D, int max_len, long k_sb, long k_sh, float scale, void *work, unsigned *ctr,
                            hipStream_t s, int o_packed_d, bool kv_bf16 = false, bool wide = false);
// key splits attn_decode_impl launches for this shape (1: one pass, no merge; 0: bad shape)
int attn_decode_splits(int B, int H, int D, int max_len, bool kv_bf16, bool wide);


// two-pass row argmax with caller-provided scratch of argmax_workspace_bytes(n, V) bytes
size_t argmax_workspace_bytes(int n, int V);
jas_status argmax_impl(const float *x, int n, int V, long ld, int32_t *out, void *work, hipStream_t s);

#define JAS_HIP(expr)                                                                 \
    do {                                                                              \
        hipError_t e_ = (expr);                                                       \
        if (e_ != hipSuccess)                                                         \
            return ::jas::fail(JAS_ERR_HIP, std::string(#expr ": ") + hipGetErrorString(e_)); \
    } while (0)

#define JAS_CHECK(cond, code, msg)                                                    \
    do {                                                                              \
        if (!(cond)) return ::jas::fail(code, msg);                                   \
    } while (0)

#define JAS_LAUNCH_CHECK() JAS_HIP(hipGetLastError())

constexpr int WAVE = 64;

// fp32 -> bf16, round to nearest even (NaN stays a quiet NaN of the same sign)
__host__ __device__ inline uint16_t f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__host__ __device__ inline float bf16_to_f32(uint16_t v)
{
    const uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// four consecutive bf16 elements (one 8-byte load) widened to fp32
__device__ __forceinline__ floatx4 widen_bf16x4(u32x2 u)
{
    return floatx4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                   __uint_as_float(u.y & 0xffff0000u)};
}

// ---- wave64 reductions in registers ----
// Partners meet through DPP within a 16-lane row (quad permutes lane ^ 1 and lane ^ 2, then
// the half-row and row mirrors) and through the gfx950 row swaps across rows
// (v_permlane16_swap, v_permlane32_swap) -- no LDS permutes.  Every step combines two values
// in either order, so all 64 lanes end with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op)
{
    v = op(v, dpp_f32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = op(v, dpp_f32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = op(v, dpp_f32<0x141>(v));  // row_half_mirror
    v = op(v, dpp_f32<0x140>(v));  // row_mirror
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float wave_sum(float v)
{
    return wave_reduce(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v)
{
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ double wave_sum_d(double v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// block-wide reduction through LDS; every thread gets the result.  `red` holds >= 16 floats.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float *red)
{
    v = wave_sum(v);
    constexpr int NW = NT / WAVE;
    if (NW == 1) return v;
    int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) s += red[i];
    return s;
}
template <int NT>
__device__ __forceinline__ float block_max(float v, float *red)
{
    v = wave_max(v);
    constexpr int NW = NT / WAVE;
    if (NW == 1) return v;
    int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) s = fmaxf(s, red[i]);
    return s;
}

// GPT-2 tanh GELU and SiLU in fp32
__device__ __forceinline__ float gelu_f(float x)
{
#pragma clang fp contract(fast)
    float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanhf(u));
}
__device__ __forceinline__ double gelu_d(double x)
{
#pragma clang fp contract(fast)
    return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
}
__device__ __forceinline__ float silu_f(float x)
{
#pragma clang fp contract(fast)
    return x / (1.0f + expf(-x));
}

__device__ __forceinline__ float apply_act(float v, int act)
{
    switch (act) {
    case JAS_ACT_RELU: return (float)(v > 0.0f) * v;  // (x>0)*x keeps jasmine's -0 / NaN
    case JAS_ACT_GELU: return gelu_f(v);
    case JAS_ACT_SILU: return silu_f(v);
    case JAS_ACT_SIGMOID: return (float)(1.0 / (1.0 + (double)expf(-v)));
    default: return v;
    }
}

inline unsigned ceil_div(long a, long b) { return (unsigned)((a + b - 1) / b); }

// counter-based N(mean,std): splitmix64 + Box-Muller, identical formula on host and device
__host__ __device__ inline uint64_t splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
__host__ __device__ inline uint64_t stream_key(uint64_t seed, uint64_t stream)
{
    return splitmix64(splitmix64(seed) ^ (stream * 0xD1B54A32D192ED03ull));
}

} // namespace jas
