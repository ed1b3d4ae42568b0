// Attention (north-star item 4): flash-attention prefill and split-K KV-cache decode.
//
// Reference: mat_head_gen_t::forward (mat_mha_t.hpp:45-74) materialises the full
// S = Q'K / sqrt(d) matrix, masks j > i to -inf (:58-67), runs hsoftmax and multiplies
// V P'.  Decoding (test_transformer_t::predict, transformer_test.hpp:194-242) recomputes
// the whole prefix every step.  Here:
//  * prefill never materialises S: each workgroup owns 64 queries (16 per wave), streams
//    64-key K/V tiles through LDS and keeps an online softmax.  The wave computes
//    S^T = K Q^T with v_mfma_f32_16x16x4_f32 so that the probabilities land in exactly the
//    B-operand layout of the O^T += V^T P^T product -- P never leaves registers.
//  * decode splits each (sequence, head)'s keys over workgroups (flash-decoding), each
//    reading its K/V slice once from HBM, then merges the partial softmaxes by log-sum-exp.
#include "jas_common.hpp"

#include <cfloat>

namespace jas {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t v)
{
    return __uint_as_float((uint32_t)v << 16);
}

template <bool BF16>
__device__ __forceinline__ float4 load4(const void *base, long idx)
{
    if (BF16) {
        uint2 u = *(const uint2 *)((const uint16_t *)base + idx);
        return make_float4(bf16_to_f32(u.x & 0xffff), bf16_to_f32(u.x >> 16), bf16_to_f32(u.y & 0xffff),
                           bf16_to_f32(u.y >> 16));
    }
    return *(const float4 *)((const float *)base + idx);
}

template <bool BF16>
__device__ __forceinline__ void store4(void *base, long idx, float4 v)
{
    if (BF16) {
        auto cvt = [](float f) -> uint32_t {  // round to nearest even
            uint32_t u = __float_as_uint(f);
            if ((u & 0x7fffffff) > 0x7f800000) return 0x7fc0;
            return (u + 0x7fff + ((u >> 16) & 1)) >> 16;
        };
        uint2 o;
        o.x = cvt(v.x) | (cvt(v.y) << 16);
        o.y = cvt(v.z) | (cvt(v.w) << 16);
        *(uint2 *)((uint16_t *)base + idx) = o;
    } else {
        *(float4 *)((float *)base + idx) = v;
    }
}

struct PrefillArgs {
    const void *Q, *K, *V;
    void *O;
    long q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, o_sb, o_sh, o_ss;
    int B, H, Sq, Sk;
    float scale_log2;  // scale * log2(e)
    int causal;
};

constexpr int FA_BQ = 64, FA_BK = 64;

template <int D, bool BF16>
__global__ void __launch_bounds__(256) flash_prefill_kernel(const PrefillArgs p)
{
    constexpr int KLD = D + 4;        // Ks row stride
    constexpr int VLD = FA_BK + 4;    // Vt row stride
    constexpr int NC = D / 16;        // 16-wide chunks of the head dim
    __shared__ float Ks[FA_BK * KLD];
    __shared__ float Vt[D * VLD];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g = lane >> 4;
    const int nqb = (p.Sq + FA_BQ - 1) / FA_BQ;
    const int qb = nqb - 1 - (int)blockIdx.x;  // heaviest (causal) query blocks first
    const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
    const int q0 = qb * FA_BQ + w * 16;
    const int qi = q0 + r16;  // this lane's query (column of S^T)
    const int shift = p.Sk - p.Sq;

    const char *Qb = (const char *)p.Q;
    // Q fragment: lane holds Q[qi][16c + 4g .. +3], prescaled by scale*log2(e)
    float4 qf[NC];
    {
        const int qq = qi < p.Sq ? qi : p.Sq - 1;
        long base = (long)b * p.q_sb + (long)h * p.q_sh + (long)qq * p.q_ss;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float4 v = load4<BF16>(Qb, base + 16 * c + 4 * g);
            qf[c] = make_float4(v.x * p.scale_log2, v.y * p.scale_log2, v.z * p.scale_log2, v.w * p.scale_log2);
        }
    }

    floatx4 oacc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) oacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -FLT_MAX, l_run = 0.f;

    const int q_last = min(qb * FA_BQ + FA_BQ - 1, p.Sq - 1);
    const int k_end = p.causal ? min(p.Sk, q_last + shift + 1) : p.Sk;
    const long kbase = (long)b * p.k_sb + (long)h * p.k_sh;

    for (int kv0 = 0; kv0 < k_end; kv0 += FA_BK) {
        __syncthreads();
        // stage K (row-major) and V (transposed) tiles: 64 keys x D
#pragma unroll
        for (int it = 0; it < (FA_BK * D / 4) / 256; ++it) {
            int idx = tid + it * 256;
            int key = idx / (D / 4), d4 = (idx % (D / 4)) * 4;
            int kk = kv0 + key;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (kk < p.Sk) {
                kv = load4<BF16>(p.K, kbase + (long)kk * p.k_ss + d4);
                vv = load4<BF16>(p.V, kbase + (long)kk * p.k_ss + d4);
            }
            *(float4 *)(Ks + key * KLD + d4) = kv;
            Vt[(d4 + 0) * VLD + key] = vv.x;
            Vt[(d4 + 1) * VLD + key] = vv.y;
            Vt[(d4 + 2) * VLD + key] = vv.z;
            Vt[(d4 + 3) * VLD + key] = vv.w;
        }
        __syncthreads();

        // S^T tile: lane holds S^T[key = 16j + 4g + r][query = qi]
        floatx4 s[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float4 kf = *(const float4 *)(Ks + (16 * j + r16) * KLD + 16 * c + 4 * g);
                s[j] = mfma4(kf.x, qf[c].x, s[j]);
                s[j] = mfma4(kf.y, qf[c].y, s[j]);
                s[j] = mfma4(kf.z, qf[c].z, s[j]);
                s[j] = mfma4(kf.w, qf[c].w, s[j]);
            }
        }
        // mask and tile max for this lane's query
        float tmax = -FLT_MAX;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int kk = kv0 + 16 * j + 4 * g + r;
                bool ok = kk < p.Sk && (!p.causal || kk <= qi + shift);
                s[j][r] = ok ? s[j][r] : -FLT_MAX;
                tmax = fmaxf(tmax, s[j][r]);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, WAVE));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, WAVE));
        const float m_new = fmaxf(m_run, tmax);
        const float corr = exp2f(m_run - m_new);
        float psum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float pv = s[j][r] == -FLT_MAX ? 0.f : exp2f(s[j][r] - m_new);
                s[j][r] = pv;
                psum += pv;
            }
        psum += __shfl_xor(psum, 16, WAVE);
        psum += __shfl_xor(psum, 32, WAVE);
        l_run = l_run * corr + psum;
        m_run = m_new;
#pragma unroll
        for (int c = 0; c < NC; ++c) oacc[c] *= corr;
        // O^T[d = 16c + 4g + r][q] += sum_key V^T[d][key] P^T[key][q]
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float4 vf = *(const float4 *)(Vt + (16 * c + r16) * VLD + 16 * j + 4 * g);
                oacc[c] = mfma4(vf.x, s[j][0], oacc[c]);
                oacc[c] = mfma4(vf.y, s[j][1], oacc[c]);
                oacc[c] = mfma4(vf.z, s[j][2], oacc[c]);
                oacc[c] = mfma4(vf.w, s[j][3], oacc[c]);
            }
    }

    // lane holds O^T[d = 16c + 4g + r][query = qi], i.e. four consecutive dims of its query
    if (qi < p.Sq) {
        const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
        long obase = (long)b * p.o_sb + (long)h * p.o_sh + (long)qi * p.o_ss;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            store4<BF16>(p.O, obase + 16 * c + 4 * g,
                         make_float4(oacc[c][0] * inv, oacc[c][1] * inv, oacc[c][2] * inv, oacc[c][3] * inv));
    }
}

// ---------------------------------------------------------------- decode
struct DecodeArgs {
    const float *q, *K, *V;
    float *O;
    const int32_t *seqlens;
    float *part;  // [B*H][nsplit][D + 2]
    long k_sb, k_sh;
    int B, H, nsplit, chunk;
    float scale_log2;
    int o_packed_d;  // > 0: write O in the packed B-operand layout over o_packed_d features
};

__device__ __forceinline__ long decode_out_index(const DecodeArgs &p, int bh, int D, int e)
{
    if (p.o_packed_d <= 0) return (long)bh * D + e;
    const int b = bh / p.H, k = (bh % p.H) * D + e;  // token b, feature k
    return ((long)(k >> 4) * 64 + b + 16 * ((k & 15) >> 2)) * 4 + (k & 3);
}

// TPK lanes per key (D/4 floats each); each group of TPK lanes walks its own keys.
template <int D>
__global__ void __launch_bounds__(256) attn_decode_kernel(const DecodeArgs p)
{
    constexpr int TPK = D / 4;              // lanes per key
    constexpr int GPW = WAVE / TPK;         // key groups per wave
    constexpr int NG = 4 * GPW;             // key groups per workgroup
    constexpr int U = 4;                    // keys per group per iteration (loads in flight)
    __shared__ float sm[NG], sl[NG];
    __shared__ float sacc[NG][D];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int grp = w * GPW + lane / TPK, lig = lane % TPK;
    const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H, split = blockIdx.x;
    const int len = p.seqlens[b];
    const int k0 = split * p.chunk, k1 = min(len, k0 + p.chunk);

    float4 q = *(const float4 *)(p.q + (long)bh * D + 4 * lig);
    q.x *= p.scale_log2; q.y *= p.scale_log2; q.z *= p.scale_log2; q.w *= p.scale_log2;
    const float *Kb = p.K + (long)b * p.k_sb + (long)h * p.k_sh + 4 * lig;
    const float *Vb = p.V + (long)b * p.k_sb + (long)h * p.k_sh + 4 * lig;

    float m = -FLT_MAX, l = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int kk = k0 + grp; kk < k1; kk += NG * U) {
        floatx4 kv[U], vv[U];
        float sc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int key = kk + u * NG;
            bool ok = key < k1;
            kv[u] = ok ? __builtin_nontemporal_load((const floatx4 *)(Kb + (long)key * D)) : floatx4{0.f, 0.f, 0.f, 0.f};
            vv[u] = ok ? __builtin_nontemporal_load((const floatx4 *)(Vb + (long)key * D)) : floatx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float d = q.x * kv[u][0] + q.y * kv[u][1] + q.z * kv[u][2] + q.w * kv[u][3];
#pragma unroll
            for (int o = TPK / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, WAVE);
            sc[u] = (kk + u * NG) < k1 ? d : -FLT_MAX;
        }
        float mx = m;
#pragma unroll
        for (int u = 0; u < U; ++u) mx = fmaxf(mx, sc[u]);
        float corr = exp2f(m - mx);
        l *= corr;
        acc.x *= corr; acc.y *= corr; acc.z *= corr; acc.w *= corr;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float pv = sc[u] == -FLT_MAX ? 0.f : exp2f(sc[u] - mx);
            l += pv;
            acc.x += pv * vv[u][0]; acc.y += pv * vv[u][1]; acc.z += pv * vv[u][2]; acc.w += pv * vv[u][3];
        }
        m = mx;
    }
    // merge the key groups of this workgroup
    if (lig == 0) { sm[grp] = m; sl[grp] = l; }
    *(float4 *)(&sacc[grp][4 * lig]) = acc;
    __syncthreads();
    if (tid < D) {
        float M = -FLT_MAX;
#pragma unroll
        for (int k = 0; k < NG; ++k) M = fmaxf(M, sm[k]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            float f = sm[k] == -FLT_MAX ? 0.f : exp2f(sm[k] - M);
            L += sl[k] * f;
            A += sacc[k][tid] * f;
        }
        if (p.nsplit == 1) {
            p.O[decode_out_index(p, bh, D, tid)] = L > 0.f ? A / L : 0.f;
        } else {
            float *pp = p.part + ((long)bh * p.nsplit + split) * (D + 2);
            pp[2 + tid] = A;
            if (tid == 0) { pp[0] = M; pp[1] = L; }
        }
    }
}

template <int D>
__global__ void __launch_bounds__(D) attn_decode_merge_kernel(const DecodeArgs p)
{
    const int bh = blockIdx.x, tid = threadIdx.x;
    const float *pp = p.part + (long)bh * p.nsplit * (D + 2);
    float M = -FLT_MAX;
    for (int s = 0; s < p.nsplit; ++s) M = fmaxf(M, pp[s * (D + 2)]);
    float L = 0.f, A = 0.f;
    for (int s = 0; s < p.nsplit; ++s) {
        float ms = pp[s * (D + 2)];
        float f = ms == -FLT_MAX ? 0.f : exp2f(ms - M);
        L += pp[s * (D + 2) + 1] * f;
        A += pp[s * (D + 2) + 2 + tid] * f;
    }
    p.O[decode_out_index(p, bh, D, tid)] = L > 0.f ? A / L : 0.f;
}

static int decode_nsplit(int B, int H, int D, int max_len, int *chunk)
{
    const int keys_per_step = 4 * (WAVE / (D / 4)) * 4;  // NG * U
    int pairs = B * H;
    int want = (2048 + pairs - 1) / pairs;
    int max_split = (max_len + keys_per_step - 1) / keys_per_step;
    int ns = std::max(1, std::min(want, max_split));
    int ch = (max_len + ns - 1) / ns;
    ch = ((ch + keys_per_step - 1) / keys_per_step) * keys_per_step;
    ns = std::max(1, (max_len + ch - 1) / ch);
    *chunk = ch;
    return ns;
}

jas_status attn_decode_impl(const float *q, const float *K, const float *V, float *O, const int32_t *seqlens, int B,
                            int H, int D, int max_len, long k_sb, long k_sh, float scale, void *work, hipStream_t s,
                            int o_packed_d)
{
    JAS_CHECK(q && K && V && O && seqlens, JAS_ERR_INVALID, "jas_attn_decode: null tensor");
    JAS_CHECK(B > 0 && H > 0 && max_len > 0, JAS_ERR_INVALID, "jas_attn_decode: empty shape");
    JAS_CHECK(D == 32 || D == 64 || D == 128, JAS_ERR_INVALID, "jas_attn_decode: head dim must be 32, 64 or 128");
    JAS_CHECK(k_sb % 4 == 0 && k_sh % 4 == 0, JAS_ERR_INVALID, "jas_attn_decode: strides must be multiples of 4");
    int chunk;
    int ns = decode_nsplit(B, H, D, max_len, &chunk);
    JAS_CHECK(ns == 1 || work, JAS_ERR_INVALID, "jas_attn_decode: workspace required");
    JAS_CHECK(o_packed_d <= 0 || (B <= 16 && o_packed_d == H * D), JAS_ERR_INVALID, "attn_decode: bad packed output");
    DecodeArgs p{q, K, V, O, seqlens, (float *)work, k_sb, k_sh, B, H, ns, chunk, scale * 1.4426950408889634f,
                 o_packed_d};
    dim3 grid(ns, B * H);
#define JAS_DEC(DD)                                                                                  \
    if (D == DD) {                                                                                   \
        hipLaunchKernelGGL((attn_decode_kernel<DD>), grid, dim3(256), 0, s, p);                      \
        if (ns > 1) hipLaunchKernelGGL((attn_decode_merge_kernel<DD>), dim3(B * H), dim3(DD), 0, s, p); \
    }
    JAS_DEC(32) JAS_DEC(64) JAS_DEC(128)
#undef JAS_DEC
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}


} // namespace jas

using namespace jas;

extern "C" {

jas_status jas_attn_prefill(const void *Q, const void *K, const void *V, void *O, int B, int H, int Sq, int Sk, int D,
                            long q_sb, long q_sh, long q_ss, long k_sb, long k_sh, long k_ss, long o_sb, long o_sh,
                            long o_ss, float scale, int causal, int dtype, jas_stream_t stream)
{
    JAS_CHECK(Q && K && V && O, JAS_ERR_INVALID, "jas_attn_prefill: null tensor");
    JAS_CHECK(B > 0 && H > 0 && Sq > 0 && Sk > 0, JAS_ERR_INVALID, "jas_attn_prefill: empty shape");
    JAS_CHECK(D == 32 || D == 64 || D == 128, JAS_ERR_INVALID, "jas_attn_prefill: head dim must be 32, 64 or 128");
    JAS_CHECK(dtype == JAS_F32 || dtype == JAS_BF16, JAS_ERR_INVALID, "jas_attn_prefill: dtype f32 or bf16");
    JAS_CHECK(!causal || Sk >= Sq, JAS_ERR_INVALID, "jas_attn_prefill: causal needs Sk >= Sq");
    const long al = 4;  // every access is a 4-element vector (16 B f32, 8 B bf16)
    JAS_CHECK(q_ss % al == 0 && k_ss % al == 0 && o_ss % al == 0 && q_sh % al == 0 && k_sh % al == 0 &&
                  o_sh % al == 0 && q_sb % al == 0 && k_sb % al == 0 && o_sb % al == 0,
              JAS_ERR_INVALID, "jas_attn_prefill: strides must be multiples of 4 elements");
    PrefillArgs p{Q, K, V, O, q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, o_sb, o_sh, o_ss, B, H, Sq, Sk,
                  scale * 1.4426950408889634f, causal};
    dim3 grid(ceil_div(Sq, FA_BQ), B * H);
    hipStream_t s = stream_or_default(stream);
#define JAS_FA(DD)                                                                                         \
    if (D == DD) {                                                                                         \
        if (dtype == JAS_BF16) hipLaunchKernelGGL((flash_prefill_kernel<DD, true>), grid, dim3(256), 0, s, p); \
        else hipLaunchKernelGGL((flash_prefill_kernel<DD, false>), grid, dim3(256), 0, s, p);               \
    }
    JAS_FA(32) JAS_FA(64) JAS_FA(128)
#undef JAS_FA
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

size_t jas_attn_decode_workspace(int B, int H, int D, int max_len)
{
    if (B <= 0 || H <= 0 || max_len <= 0 || (D != 32 && D != 64 && D != 128)) return 0;
    int chunk;
    int ns = decode_nsplit(B, H, D, max_len, &chunk);
    return ns > 1 ? sizeof(float) * (size_t)B * H * ns * (D + 2) : 0;
}

jas_status jas_attn_decode(const float *q, const float *K, const float *V, float *O, const int32_t *seqlens, int B,
                           int H, int D, int max_len, long k_sb, long k_sh, float scale, void *work,
                           jas_stream_t stream)
{
    return attn_decode_impl(q, K, V, O, seqlens, B, H, D, max_len, k_sb, k_sh, scale, work, stream_or_default(stream), 0);
}

} // extern "C"
