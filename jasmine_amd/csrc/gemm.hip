// fp32 GEMMs on the CDNA4 matrix cores.
//
// Reference: mat_dot_t::operator() (mat_express_t.hpp:730-736) is a scalar triple loop
// with sequential-k accumulation, reached from weight_net_t::forward (mat_net_t.hpp:38-49)
// for every projection and from mat_head_gen_t::forward (mat_mha_t.hpp:53,71).
//
// Two kernels:
//  * gemm_tile_kernel: 128x128x16 LDS-tiled MFMA GEMM (v_mfma_f32_16x16x4_f32) for
//    prefill-sized problems; any operand strides (transposed views included).
//  * skinny_kernel: N <= 16 tokens (decode).  The weight matrix is streamed from HBM
//    straight into MFMA A-operand registers (no LDS), one 16-row tile per wave set, the
//    K range split across the waves of a workgroup and reduced through LDS, with the
//    layer's elementwise tail fused into the epilogue (bias, GELU, residual add, SwiGLU,
//    RoPE + KV-cache append).
//
// MFMA 16x16x4 f32 operand layout (lane l of 64): A[i = l%16][kslot = l/16],
// B[kslot = l/16][j = l%16], D rows 4*(l/16)+r (r = 0..3), column l%16.  Each lane loads
// a float4 along K; sub-step t of 4 feeds element t, so k-slot s of sub-step t is
// k = 4s + t -- a permutation of K applied identically to A and B.
#include "gemm.hpp"

namespace jas {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- tiled GEMM
constexpr int TBM = 128, TBN = 128, TBK = 16;  // output tile edge, K slab width

// K-contiguous, outer-contiguous, generic strides, packed weights (weight_pack_offset)
// and the packed layout with bf16 elements (widened on load)
enum LoadMode : int { LM_KC = 0, LM_OC = 1, LM_GEN = 2, LM_PK = 3, LM_PKB = 4 };


// Loads an [OUTER (128 or 64) outer x KW (16 or 32) k] tile of X(o, k) = X[o*so + k*sk]
// into registers (256 threads), then LDS rows [o][k] (K-contiguous, padded stride KW + 4).
// The packed layouts are read in 16-wide K blocks only.
template <int MODE, int OUTER = 128, int KW = 16>
struct TileLoader {
    static_assert(KW == 16 || (MODE != LM_PK && MODE != LM_PKB), "packed operands use 16-wide K slabs");
    static constexpr int LD = KW + 4;              // LDS row stride (floats)
    static constexpr int NV = OUTER * KW / 1024;   // float4 loads per thread (vector modes)
    static constexpr int NS = OUTER * KW / 256;    // scalar loads per thread (generic mode)
    float r[NS];
    __device__ __forceinline__ void load(const float *__restrict__ X, long so, long sk, int o0, int k0, int O, int K,
                                         int tid)
    {
        if (MODE == LM_KC) {
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                int idx = tid + q * 256, o = idx / (KW / 4), kq = (idx % (KW / 4)) * 4;
                int go = o0 + o, gk = k0 + kq;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (go < O && gk < K) v = *(const float4 *)(X + (long)go * so + gk);
                r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
            }
        } else if (MODE == LM_PK || MODE == LM_PKB) {  // 8 row tiles x one 16-wide K block: 8 contiguous blocks
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                int idx = tid + q * 256, i = idx >> 6, ln = idx & 63;
                long rt = o0 / 16 + i;
                floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
                if (rt * 16 < O) {
                    if (MODE == LM_PKB) {  // half (k0/16)%2 of the pair tile: 4 of the lane's 8 elements
                        const int kb = k0 >> 4;
                        const long off = weight_tile_offset_b(rt, kb >> 1, k32_of(K), (O + 15) >> 4) + ln * 8 + 4 * (kb & 1);
                        v = widen_bf16x4(*(const u32x2 *)((const uint16_t *)(const void *)X + off));
                    } else {
                        v = *(const floatx4 *)(X + weight_tile_offset(rt, k0 >> 4, K >> 4, (O + 15) >> 4) + ln * 4);
                    }
                }
                r[4 * q] = v[0]; r[4 * q + 1] = v[1]; r[4 * q + 2] = v[2]; r[4 * q + 3] = v[3];
            }
        } else if (MODE == LM_OC) {
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                int idx = tid + q * 256, k = idx / (OUTER / 4), oq = (idx % (OUTER / 4)) * 4;
                int go = o0 + oq, gk = k0 + k;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (go < O && gk < K) v = *(const float4 *)(X + (long)gk * sk + go);
                r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                int idx = tid + q * 256, o = idx / KW, k = idx % KW;
                int go = o0 + o, gk = k0 + k;
                r[q] = (go < O && gk < K) ? X[(long)go * so + (long)gk * sk] : 0.f;
            }
        }
    }
    __device__ __forceinline__ void store(float *lds, int tid) const
    {
        if (MODE == LM_KC) {
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                int idx = tid + q * 256, o = idx / (KW / 4), kq = (idx % (KW / 4)) * 4;
                *(float4 *)(lds + o * LD + kq) = make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
            }
        } else if (MODE == LM_PK || MODE == LM_PKB) {
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                int idx = tid + q * 256, i = idx >> 6, ln = idx & 63;
                *(float4 *)(lds + (i * 16 + (ln & 15)) * LD + 4 * (ln >> 4)) =
                    make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
            }
        } else if (MODE == LM_OC) {
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                int idx = tid + q * 256, k = idx / (OUTER / 4), oq = (idx % (OUTER / 4)) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) lds[(oq + e) * LD + k] = r[4 * q + e];
            }
        } else {
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                int idx = tid + q * 256, o = idx / KW, k = idx % KW;
                lds[o * LD + k] = r[q];
            }
        }
    }
};

struct TileArgs {
    const float *A, *B;
    float *C;
    const float *bias;
    long as0, as1, bs0, bs1, cs0, cs1;
    long abs_, bbs, cbs, biasbs;
    int M, N, K;
    int bias_mode, act, accumulate;
};

// T x T output tile (T = 128, or 64 for problems too small to fill the chip with 128-wide
// tiles); 4 waves in a 2 x 2 grid, each T/2 x T/2 (NB x NB blocks of 16 x 16)
template <int AM, int BMODE, bool C4, int T = TBM, int KW = TBK>
__global__ void __launch_bounds__(256) gemm_tile_kernel(const TileArgs p)
{
    constexpr int NB = T / 32, LD = KW + 4;
    // two LDS buffers: slab k is read from one while slab k+1 is written to the other
    __shared__ float As[2][T * LD];
    __shared__ float Bs[2][T * LD];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w >> 1, wn = w & 1, r16 = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * T, n0 = blockIdx.x * T;
    const long bz = blockIdx.z;
    const float *A = p.A + bz * p.abs_;
    const float *B = p.B + bz * p.bbs;
    float *C = p.C + bz * p.cbs;
    const float *bias = p.bias ? p.bias + bz * p.biasbs : nullptr;

    TileLoader<AM, T, KW> la;
    TileLoader<BMODE, T, KW> lb;
    // A(m, k) = A[m*as0 + k*as1]: outer = m.  B(k, n) = B[k*bs0 + n*bs1]: outer = n.
    la.load(A, p.as0, p.as1, m0, 0, p.M, p.K, tid);
    lb.load(B, p.bs1, p.bs0, n0, 0, p.N, p.K, tid);
    la.store(As[0], tid);
    lb.store(Bs[0], tid);
    if (KW < p.K) {  // slab 1 in flight
        la.load(A, p.as0, p.as1, m0, KW, p.M, p.K, tid);
        lb.load(B, p.bs1, p.bs0, n0, KW, p.N, p.K, tid);
    }
    __syncthreads();

    floatx4 acc[NB][NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    int buf = 0;
    for (int k0 = 0; k0 < p.K; k0 += KW) {
        // stage slab k+1 (in registers) into the other buffer, then start slab k+2's loads;
        // the other buffer was last read in the previous step, before its closing barrier
        if (k0 + KW < p.K) {
            la.store(As[buf ^ 1], tid);
            lb.store(Bs[buf ^ 1], tid);
            if (k0 + 2 * KW < p.K) {
                la.load(A, p.as0, p.as1, m0, k0 + 2 * KW, p.M, p.K, tid);
                lb.load(B, p.bs1, p.bs0, n0, k0 + 2 * KW, p.N, p.K, tid);
            }
        }
        const float *as = As[buf], *bs = Bs[buf];
#pragma unroll
        for (int kh = 0; kh < KW / 16; ++kh) {  // 16-wide K blocks of the slab
            float4 a[NB], b[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i)
                a[i] = *(const float4 *)(as + (wm * (T / 2) + i * 16 + r16) * LD + 16 * kh + 4 * g);
#pragma unroll
            for (int j = 0; j < NB; ++j)
                b[j] = *(const float4 *)(bs + (wn * (T / 2) + j * 16 + r16) * LD + 16 * kh + 4 * g);
#pragma unroll
            for (int i = 0; i < NB; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    acc[i][j] = mfma4(a[i].x, b[j].x, acc[i][j]);
                    acc[i][j] = mfma4(a[i].y, b[j].y, acc[i][j]);
                    acc[i][j] = mfma4(a[i].z, b[j].z, acc[i][j]);
                    acc[i][j] = mfma4(a[i].w, b[j].w, acc[i][j]);
                }
        }
        __syncthreads();
        buf ^= 1;
    }

    // epilogue: lane holds rows m = 4g + r of each 16x16 block, column n = r16
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int mb = m0 + wm * (T / 2) + i * 16 + 4 * g, n = n0 + wn * (T / 2) + j * 16 + r16;
            if (n >= p.N) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int m = mb + r;
                float x = acc[i][j][r];
                if (bias && m < p.M) x = x + (p.bias_mode == 1 ? bias[m] : bias[n]);
                v[r] = apply_act(x, p.act);
            }
            float *cp = C + (long)mb * p.cs0 + (long)n * p.cs1;
            if (C4 && mb + 3 < p.M) {  // cs0 == 1: four consecutive rows are contiguous
                float4 o = make_float4(v[0], v[1], v[2], v[3]);
                if (p.accumulate) {
                    float4 c = *(float4 *)cp;
                    o.x += c.x; o.y += c.y; o.z += c.z; o.w += c.w;
                }
                *(float4 *)cp = o;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (mb + r < p.M) {
                        float *q = cp + (long)r * p.cs0;
                        *q = p.accumulate ? *q + v[r] : v[r];
                    }
            }
        }
}

// 64-wide tiles of plain operands take K slabs of 32 (128-byte row segments, half the
// barriers per flop); 128-wide tiles keep 16 (32-wide slabs need 72 KB of LDS there and
// lose occupancy), as do packed weights
template <int AM, int BMODE>
static void launch_tile_c(const TileArgs &p, bool c4, bool small, int batch, hipStream_t s)
{
    constexpr int KW = (AM == LM_PK || AM == LM_PKB) ? 16 : 32;
    if (small) {
        const dim3 grid(ceil_div(p.N, 64), ceil_div(p.M, 64), batch);
        if (c4) hipLaunchKernelGGL((gemm_tile_kernel<AM, BMODE, true, 64, KW>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_tile_kernel<AM, BMODE, false, 64, KW>), grid, dim3(256), 0, s, p);
    } else {
        const dim3 grid(ceil_div(p.N, TBN), ceil_div(p.M, TBM), batch);
        if (c4) hipLaunchKernelGGL((gemm_tile_kernel<AM, BMODE, true, TBM, TBK>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_tile_kernel<AM, BMODE, false, TBM, TBK>), grid, dim3(256), 0, s, p);
    }
}

template <int AM>
static void launch_tile_b(const TileArgs &p, int bm, bool c4, bool small, int batch, hipStream_t s)
{
    if (bm == LM_KC) launch_tile_c<AM, LM_KC>(p, c4, small, batch, s);
    else if (bm == LM_OC) launch_tile_c<AM, LM_OC>(p, c4, small, batch, s);
    else launch_tile_c<AM, LM_GEN>(p, c4, small, batch, s);
}

static bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// choose a vector load mode for operand X(o, k) = X[o*so + k*sk] over a batch
static int pick_mode(const float *X, long so, long sk, int O, int K, long bstride)
{
    bool base = al16(X) && (bstride % 4 == 0);
    if (sk == 1 && K % 4 == 0 && so % 4 == 0 && base) return LM_KC;
    if (so == 1 && O % 4 == 0 && sk % 4 == 0 && base) return LM_OC;
    return LM_GEN;
}

// ---------------------------------------------------------------- direct-to-LDS GEMM
// The main fp32 GEMM for operands that are contiguous in one dimension.  K slabs of
// 16 * KB are moved from global memory straight into LDS (global_load_lds_dwordx4: each
// wave instruction writes 64 lanes x 16 B contiguously at a wave-uniform LDS base), so no
// register staging and no LDS store instructions sit in the loop.  ST stage buffers keep
// ST - 1 slabs in flight; one barrier per slab.
//
// LDS layouts, chosen so that every fragment read is one conflict-free ds_read_b128:
//  * K-contiguous operand X(o, k) (and the packed weight layout): per 16 x 16 block, the 64
//    lanes' float4s in MFMA operand order -- lane r + 16 g holds X(16 b + r, 4 g .. 4 g + 3).
//    Sub-step t of the four 16x16x4 MFMAs per block takes element t, so k-slot g of
//    sub-step t is k = 4 g + t, a permutation of K applied to both operands alike.
//  * Outer-contiguous operand: rows [k][o] as in memory.  Lane (g, r) reads the float4
//    X(o0 + 4 r .. 4 r + 3, k = 4 g + t): its four elements feed four different 16-wide
//    blocks (block e takes outer index 4 r + e), so one read serves four MFMAs, and the
//    output of those blocks comes out as four consecutive columns per lane.
// The compiler cannot see the LDS writes of the DMA (they are issued as asm, so its
// wait-count pass does not serialise the LDS reads behind every load in flight); the loop
// waits on vmcnt itself before each barrier.
enum DmaMode : int { DM_KC = 0, DM_OC = 1, DM_PK = 2 };

struct DmaArgs {
    const float *A, *B;
    float *C;
    const float *bias;
    long as0, as1, bs0, bs1, cs0, cs1;
    long abs_, bbs, cbs, biasbs;
    int M, N, K;
    int bias_mode, act, accumulate;
    int c_vec;  // 1: row-major C with float4 stores over n; 2: column-major C, float4 over m
    // fused prefill epilogues (packed weights, token-major output, c_vec == 2)
    DmaFused fz;
    // residual source added after the bias (residual_net_t's f(x) + x): R(m, n) = resid[m*rs0 + n*rs1]
    const float *resid = nullptr;
    long rs0 = 0, rs1 = 0;
};

// M0 is a reserved register to the compiler; nothing else in these kernels uses it (no
// relative register indexing, no other LDS DMA), which the AMD assembly of the build shows.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const float *src, float *lds_dst)
{
    const unsigned la = (unsigned)(size_t)(__attribute__((address_space(3))) float *)lds_dst;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(la), "v"(src) : "memory", "m0");
}
#pragma clang diagnostic pop

// Global address of lane `lane`'s 16 bytes for DMA instruction `ins` of the slab at k0, and
// whether the slab element group lies inside K (only the tail slab can leave K).
// X(o, k) = X[o * so + k * sk]; Olim = rows (outer extent); RG = packed row tiles.
template <int MODE, int O, int KWT>
__device__ __forceinline__ const float *dma_src(const float *X, const float *X2, long so, long sk, int o0, int Olim,
                                                int K, int k0, int ins, int lane, int &kfirst)
{
    if (MODE == DM_OC) {
        const int f = 256 * ins + 4 * lane, k = k0 + f / O;
        int o = o0 + f % O;
        o = o <= Olim - 4 ? o : Olim - 4;  // clamped groups only feed discarded outputs
        kfirst = k;
        return X + (long)(k < K ? k : K - 1) * sk + o;
    }
    constexpr int RB = O / 16;
    const int kb = ins / RB, rb = ins % RB;
    if (MODE == DM_PK) {
        const long RG = (Olim + 15) >> 4;
        long rt = min((long)(o0 >> 4) + rb, RG - 1);
        const int kblk = (k0 >> 4) + kb;
        kfirst = 16 * kblk;
        const float *Xm = X;
        long RGm = RG;
        if (X2) {  // SwiGLU: virtual row tile 2f is gate tile f, 2f + 1 up tile f
            Xm = rt & 1 ? X2 : X;
            rt >>= 1;
            RGm = RG >> 1;
        }
        return Xm + weight_tile_offset(rt, kblk < (K >> 4) ? kblk : (K >> 4) - 1, K >> 4, RGm) + lane * 4;
    }
    int o = o0 + 16 * rb + (lane & 15);
    o = o < Olim ? o : Olim - 1;
    kfirst = k0 + 16 * kb + 4 * (lane >> 4);
    return X + (long)o * so + (kfirst < K ? kfirst : 0);
}

template <int MODE, int O, int KWT, int NW>
__device__ __forceinline__ void dma_slab(const float *X, const float *X2, long so, long sk, int o0, int Olim, int K,
                                         int k0, float *lds, int w, int lane)
{
    constexpr int NI = O * KWT / 256;  // 1 KB instructions per slab
    static_assert(NI % NW == 0, "slab instructions spread evenly over the waves");
#pragma unroll
    for (int q = 0; q < NI / NW; ++q) {
        const int ins = w * (NI / NW) + q;  // wave-uniform
        int kf;
        lds_dma16(dma_src<MODE, O, KWT>(X, X2, so, sk, o0, Olim, K, k0, ins, lane, kf), lds + 256 * ins);
    }
}

// The last, partial slab (K % (16 KB) != 0): ordinary loads with zeros past K, stored in the
// same layout.
template <int MODE, int O, int KWT, int NW>
__device__ __forceinline__ void tail_slab(const float *X, const float *X2, long so, long sk, int o0, int Olim, int K,
                                          int k0, float *lds, int w, int lane)
{
    constexpr int NI = O * KWT / 256;
#pragma unroll
    for (int q = 0; q < NI / NW; ++q) {
        const int ins = w * (NI / NW) + q;
        int kf;
        const float *src = dma_src<MODE, O, KWT>(X, X2, so, sk, o0, Olim, K, k0, ins, lane, kf);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (MODE == DM_KC) {  // per element: K need not be a multiple of 4
            float e[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) e[u] = kf + u < K ? src[u] : 0.f;
            v = make_float4(e[0], e[1], e[2], e[3]);
        } else if (kf < K) {
            v = *(const float4 *)src;
        }
        *(float4 *)(lds + 256 * ins + 4 * lane) = v;
    }
}

// Fragment values of sub-step t of 16-block kb for the NB blocks of this wave
// (outer offset woff within the tile).
template <int MODE, int NB, int O>
__device__ __forceinline__ void dma_frag(const float *s, int kb, int t, int woff, int lane, float (&v)[NB],
                                         float4 (&blk)[NB])
{
    const int r16 = lane & 15, g = lane >> 4;
    if (MODE != DM_OC) {
        if (t == 0) {
#pragma unroll
            for (int i = 0; i < NB; ++i) blk[i] = *(const float4 *)(s + (kb * (O / 16) + woff / 16 + i) * 256 + lane * 4);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) v[i] = blk[i][t];
    } else {
        constexpr int G = NB < 4 ? NB : 4;
        const float *row = s + (16 * kb + 4 * g + t) * O + woff;
#pragma unroll
        for (int q = 0; q < NB / G; ++q) {
            if constexpr (G == 4) {
                const float4 x = *(const float4 *)(row + 64 * q + 4 * r16);
                v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
            } else if constexpr (G == 2) {
                const float2 x = *(const float2 *)(row + 32 * q + 2 * r16);
                v[2 * q] = x.x; v[2 * q + 1] = x.y;
            } else {
                v[q] = row[16 * q + r16];
            }
        }
    }
}

// outer index (within the wave tile) of MFMA row/column ii of block i
template <int MODE, int NB>
__device__ __forceinline__ int dma_outer(int i, int ii)
{
    constexpr int G = NB < 4 ? NB : 4;
    return MODE != DM_OC ? 16 * i + ii : 16 * G * (i / G) + G * ii + (i % G);
}

template <int N>
__device__ __forceinline__ void wait_vm_barrier()
{
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// TM x TN tile, NW waves in a WGM x (NW / WGM) grid, ST stages of 16 * KB wide K slabs.
// Workgroup ids are remapped so that each of the 8 XCDs (ids go round-robin over them)
// works on a contiguous range of tiles, walked 4 tile rows at a time: the A rows and B
// columns its workgroups share stay in that XCD's L2.
template <int AM, int BM, int TM, int TN, int NW, int WGM, int ST, int KB>
__global__ void __launch_bounds__(NW * 64) gemm_dma_kernel(const DmaArgs p)
{
    constexpr int WGN = NW / WGM, WTM = TM / WGM, WTN = TN / WGN, NBI = WTM / 16, NBJ = WTN / 16;
    constexpr int KWT = 16 * KB, SA = TM * KWT, SB = TN * KWT;
    constexpr int PER = (SA / 256 + SB / 256) / NW;  // DMA instructions per thread and slab
    static_assert(PER * (ST - 2) <= 63, "vmcnt range");
    static_assert(AM != DM_OC || NBI % 4 == 0 || NBI < 4, "outer-contiguous groups");
    __shared__ __attribute__((aligned(1024))) float lds[ST * (SA + SB)];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w / WGN, wn = w % WGN, r16 = lane & 15, g = lane >> 4;

    int bx = blockIdx.x, by = blockIdx.y;
    {
        constexpr int XG = 4;
        const int gx = gridDim.x, nt = gx * gridDim.y, per = nt / 8;
        const int id = blockIdx.y * gx + blockIdx.x;
        // a permutation of the ids: the first 8 * per go XCD-contiguous, the rest stay
        const int lid = id < 8 * per ? (id % 8) * per + id / 8 : id;
        const int grp = lid / (XG * gx), gy0 = grp * XG, rows = min(XG, (int)gridDim.y - gy0);
        const int in = lid - grp * XG * gx;
        by = gy0 + in % rows;
        bx = in / rows;
    }
    const int m0 = by * TM, n0 = bx * TN;
    const long bz = blockIdx.z;
    const float *A = p.A + bz * p.abs_;
    const float *B = p.B + bz * p.bbs;
    const int K = p.K, nk = K / KWT;
    const bool tail = nk * KWT < K;

    auto issue = [&](int kt) {
        float *sa = lds + (kt % ST) * (SA + SB), *sb = sa + SA;
        dma_slab<AM, TM, KWT, NW>(A, p.fz.A2, p.as0, p.as1, m0, p.M, K, kt * KWT, sa, w, lane);
        dma_slab<BM, TN, KWT, NW>(B, nullptr, p.bs1, p.bs0, n0, p.N, K, kt * KWT, sb, w, lane);
    };
    floatx4 acc[NBI][NBJ];
#pragma unroll
    for (int i = 0; i < NBI; ++i)
#pragma unroll
        for (int j = 0; j < NBJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const float *sa) {
        const float *sb = sa + SA;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            float4 ablk[NBI], bblk[NBJ];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float av[NBI], bv[NBJ];
                dma_frag<AM, NBI, TM>(sa, kb, t, wm * WTM, lane, av, ablk);
                dma_frag<BM, NBJ, TN>(sb, kb, t, wn * WTN, lane, bv, bblk);
#pragma unroll
                for (int i = 0; i < NBI; ++i)
#pragma unroll
                    for (int j = 0; j < NBJ; ++j) acc[i][j] = mfma4(av[i], bv[j], acc[i][j]);
            }
        }
    };

#pragma unroll
    for (int s = 0; s < ST - 1; ++s)
        if (s < nk) issue(s);
    for (int kt = 0; kt < nk; ++kt) {
        // slab kt has landed (this thread's loads: the later slabs may still be in flight);
        // the barrier makes every wave's part visible and retires the reads of the buffer
        // the next issue overwrites (last read in iteration kt - 1)
        const int ahead = min(ST - 2, nk - 1 - kt);
        if (ahead >= 2) wait_vm_barrier<2 * PER>();
        else if (ahead == 1) wait_vm_barrier<PER>();
        else wait_vm_barrier<0>();
        if (kt + ST - 1 < nk) issue(kt + ST - 1);
        compute(lds + (kt % ST) * (SA + SB));
    }
    if (tail) {
        // stage nk % ST was last read in iteration nk - ST, which every wave finished before
        // the barrier of iteration nk - 1
        float *sa = lds + (nk % ST) * (SA + SB), *sb = sa + SA;
        tail_slab<AM, TM, KWT, NW>(A, p.fz.A2, p.as0, p.as1, m0, p.M, K, nk * KWT, sa, w, lane);
        tail_slab<BM, TN, KWT, NW>(B, nullptr, p.bs1, p.bs0, n0, p.N, K, nk * KWT, sb, w, lane);
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        compute(sa);
    }

    // epilogue: block (i, j), lane (g, r16), register r holds MFMA row 4 g + r, column r16
    float *C = p.C + bz * p.cbs;
    const float *bias = p.bias ? p.bias + bz * p.biasbs : nullptr;
    auto finish = [&](float x, int m, int n, float *cp) {
        if (bias) x = x + (p.bias_mode == 1 ? bias[m] : bias[n]);
        x = apply_act(x, p.act);
        if (p.resid) x = x + p.resid[(long)m * p.rs0 + (long)n * p.rs1];
        return p.accumulate ? *cp + x : x;
    };
    const int mw = m0 + wm * WTM, nw = n0 + wn * WTN;
    if (BM == DM_OC && NBJ >= 4 && p.c_vec == 1) {  // row-major C: four consecutive n per lane
#pragma unroll
        for (int i = 0; i < NBI; ++i)
#pragma unroll
            for (int q = 0; q < NBJ / 4; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = mw + dma_outer<AM, NBI>(i, 4 * g + r), n = nw + 64 * q + 4 * r16;
                    if (m >= p.M || n >= p.N) continue;
                    float *cp = C + (long)m * p.cs0 + n;
                    float4 o;
                    o.x = finish(acc[i][4 * q][r], m, n, cp);
                    o.y = finish(acc[i][4 * q + 1][r], m, n + 1, cp + 1);
                    o.z = finish(acc[i][4 * q + 2][r], m, n + 2, cp + 2);
                    o.w = finish(acc[i][4 * q + 3][r], m, n + 3, cp + 3);
                    *(float4 *)cp = o;
                }
    } else if (AM != DM_OC && p.c_vec == 2 && p.fz.mode == FZ_SWIGLU) {
        // virtual rows: block 2k holds gate features, block 2k + 1 the up features of the same
        // 16 outputs, so both products of an output sit in one lane: out = silu(gate) * up
#pragma unroll
        for (int i = 0; i < NBI; i += 2)
#pragma unroll
            for (int j = 0; j < NBJ; ++j) {
                const int mv = mw + 16 * i + 4 * g, n = nw + dma_outer<BM, NBJ>(j, r16);
                const int f = (mv >> 5) * 16 + (mv & 15);  // output feature of this lane's first row
                if (n >= p.N || 2 * f >= p.M) continue;
                float4 o;
                o.x = silu_f(acc[i][j][0]) * acc[i + 1][j][0];
                o.y = silu_f(acc[i][j][1]) * acc[i + 1][j][1];
                o.z = silu_f(acc[i][j][2]) * acc[i + 1][j][2];
                o.w = silu_f(acc[i][j][3]) * acc[i + 1][j][3];
                *(float4 *)(C + f + (long)n * p.cs1) = o;
            }
    } else if (AM != DM_OC && p.c_vec == 2 && p.fz.mode == FZ_QKV) {
        // rows [0, d) q, [d, 2d) k, [2d, 3d) v of token n: bias, rotary on q and k (pairs
        // (2i, 2i+1) of a head are registers (0, 1) and (2, 3) of one lane), the row, and k / v
        // into the KV cache at the token's position
        const DmaFused &z = p.fz;
#pragma unroll
        for (int i = 0; i < NBI; ++i)
#pragma unroll
            for (int j = 0; j < NBJ; ++j) {
                const int m = mw + 16 * i + 4 * g, n = nw + dma_outer<BM, NBJ>(j, r16);
                if (n >= p.N || m >= p.M) continue;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = bias ? acc[i][j][r] + bias[m + r] : acc[i][j][r];
                const int sec = m / z.d, e = m % z.dh, hh = (m % z.d) / z.dh;
                const int t = z.pos[n];
                if (z.rope && sec < 2) {
#pragma unroll
                    for (int pr = 0; pr < 2; ++pr) {
                        const double2 cs = z.rope_tab[(long)t * (z.dh / 2) + (e >> 1) + pr];
                        const double x0 = v[2 * pr], x1 = v[2 * pr + 1];
                        v[2 * pr] = (float)(x0 * cs.x - x1 * cs.y);
                        v[2 * pr + 1] = (float)(x0 * cs.y + x1 * cs.x);
                    }
                }
                *(float4 *)(C + m + (long)n * p.cs1) = make_float4(v[0], v[1], v[2], v[3]);
                if (sec >= 1) {
                    const int bseq = n / z.P;
                    const long dst = (((long)bseq * z.H + hh) * z.ctx + t) * z.dh + e;
                    void *cache = sec == 1 ? z.kc : z.vc;
                    if (z.kv_bf16)
                        *(u32x2 *)((uint16_t *)cache + dst) =
                            u32x2{(uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                                  (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16)};
                    else
                        *(float4 *)((float *)cache + dst) = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
    } else if (AM != DM_OC && p.c_vec == 2) {  // column-major C: four consecutive m per lane
#pragma unroll
        for (int i = 0; i < NBI; ++i)
#pragma unroll
            for (int j = 0; j < NBJ; ++j) {
                const int m = mw + 16 * i + 4 * g, n = nw + dma_outer<BM, NBJ>(j, r16);
                if (n >= p.N || m >= p.M) continue;
                float *cp = C + m + (long)n * p.cs1;
                if (m + 3 < p.M) {
                    float4 o;
                    o.x = finish(acc[i][j][0], m, n, cp);
                    o.y = finish(acc[i][j][1], m + 1, n, cp + 1);
                    o.z = finish(acc[i][j][2], m + 2, n, cp + 2);
                    o.w = finish(acc[i][j][3], m + 3, n, cp + 3);
                    *(float4 *)cp = o;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (m + r < p.M) cp[r] = finish(acc[i][j][r], m + r, n, cp + r);
                }
            }
    } else {
#pragma unroll
        for (int i = 0; i < NBI; ++i)
#pragma unroll
            for (int j = 0; j < NBJ; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = mw + dma_outer<AM, NBI>(i, 4 * g + r), n = nw + dma_outer<BM, NBJ>(j, r16);
                    if (m >= p.M || n >= p.N) continue;
                    float *cp = C + (long)m * p.cs0 + (long)n * p.cs1;
                    *cp = finish(acc[i][j][r], m, n, cp);
                }
    }
}

// Geometry: 256 x 256 tiles (8 waves, 3 stages) when they give every CU a workgroup, else
// 128 x 128 (4 waves, 4 stages) when those give every CU at least four, else 64 x 64 (4
// waves, 4 stages of 32-wide slabs) when those give every CU one, else 32 x 32 (one 16 x 16
// block per wave: four times the workgroups; jasmine's Transformer-base encoder-decoder, 512
// x 512 products, encode 0.49 -> 0.34 ms; neutral at 1024^3).  64 x 64 tiles win wherever the 128-wide ones would
// leave a partly filled last round (GPT-2-small prefill QKV 2304 x 4096 x 768: 90 against
// 75 TFLOP/s; FC 3072 x 4096 x 768: 92 against 84).  MI355X fp32: 4096^3 at 130-137
// TFLOP/s, 2048^3 at 113, 1024^3 at 82-89.
// JAS_GEMM_GEOMETRY=256|128|64|32 forces one geometry (a tuning knob; default: the rule above).
static int forced_geometry()
{
    static const int g = [] {
        const char *e = getenv("JAS_GEMM_GEOMETRY");
        return e ? atoi(e) : 0;
    }();
    return g;
}

template <int AM, int BM>
static void launch_dma(const DmaArgs &p, int batch, hipStream_t s)
{
    auto tiles = [&](int t) { return (long)ceil_div(p.M, t) * ceil_div(p.N, t) * batch; };
    const int fg = forced_geometry();
    if (fg == 256 || (fg == 0 && tiles(256) >= 256)) {
        const dim3 grid(ceil_div(p.N, 256), ceil_div(p.M, 256), batch);
        hipLaunchKernelGGL((gemm_dma_kernel<AM, BM, 256, 256, 8, 2, 3, 1>), grid, dim3(512), 0, s, p);
    } else if (fg == 128 || (fg == 0 && tiles(128) >= 1024)) {
        const dim3 grid(ceil_div(p.N, 128), ceil_div(p.M, 128), batch);
        hipLaunchKernelGGL((gemm_dma_kernel<AM, BM, 128, 128, 4, 2, 4, 1>), grid, dim3(256), 0, s, p);
    } else if (AM != DM_PK && p.fz.mode == FZ_NONE && (fg == 32 || (fg == 0 && tiles(64) < 256))) {
        // plain operands only: packed weights and the fused prefill epilogues (SwiGLU pairs
        // two 16-row blocks in one wave) assume wave tiles of at least 32 rows
        if constexpr (AM != DM_PK) {
            const dim3 grid(ceil_div(p.N, 32), ceil_div(p.M, 32), batch);
            hipLaunchKernelGGL((gemm_dma_kernel<AM, BM, 32, 32, 4, 2, 4, 2>), grid, dim3(256), 0, s, p);
        }
    } else {
        const dim3 grid(ceil_div(p.N, 64), ceil_div(p.M, 64), batch);
        hipLaunchKernelGGL((gemm_dma_kernel<AM, BM, 64, 64, 4, 2, 4, 2>), grid, dim3(256), 0, s, p);
    }
}

// DMA load mode of operand X(o, k) = X[o * so + k * sk] (batch stride bst), or -1
static int dma_mode(const float *X, long so, long sk, int O, long bst)
{
    if (((uintptr_t)X & 15) || bst % 4) return -1;
    if (sk == 1 && so % 4 == 0) return DM_KC;
    if (so == 1 && sk % 4 == 0 && O % 4 == 0) return DM_OC;
    return -1;
}

static bool gemm_dma(int M, int N, int K, const void *A, long as0, long as1, const float *B, long bs0, long bs1,
                     float *C, long cs0, long cs1, const float *bias, int bias_mode, int act, int accumulate, int batch,
                     long abs_, long bbs, long cbs, long biasbs, hipStream_t s, bool a_packed, bool a_bf16,
                     const DmaFused *fz = nullptr, const float *resid = nullptr, long rs0 = 0, long rs1 = 0)
{
    if (a_bf16 || K <= 0) return false;
    int am = a_packed ? DM_PK : dma_mode((const float *)A, as0, as1, M, abs_);
    if (a_packed && (((uintptr_t)A & 15) || K % 16 || batch != 1)) return false;
    const int bm = dma_mode(B, bs1, bs0, N, bbs);
    if (am < 0 || bm < 0) return false;
    DmaArgs p;
    p.A = (const float *)A; p.B = B; p.C = C; p.bias = bias_mode ? bias : nullptr;
    p.as0 = as0; p.as1 = as1; p.bs0 = bs0; p.bs1 = bs1; p.cs0 = cs0; p.cs1 = cs1;
    p.abs_ = abs_; p.bbs = bbs; p.cbs = cbs; p.biasbs = biasbs;
    p.M = M; p.N = N; p.K = K;
    p.bias_mode = bias_mode; p.act = act; p.accumulate = accumulate;
    p.resid = resid; p.rs0 = rs0; p.rs1 = rs1;
    if (resid && (batch != 1 || fz)) return false;
    const bool ca = ((uintptr_t)C & 15) == 0 && cbs % 4 == 0;
    p.c_vec = 0;
    if (ca && cs1 == 1 && cs0 % 4 == 0 && N % 4 == 0) p.c_vec = 1;
    else if (ca && cs0 == 1 && cs1 % 4 == 0) p.c_vec = 2;
    if (fz) {
        if (!a_packed || p.c_vec != 2 || batch != 1 || accumulate || act != JAS_ACT_NONE) return false;
        p.fz = *fz;
    }
#define JAS_DMA_B(AMV)                                                                                 \
    if (bm == DM_KC) launch_dma<AMV, DM_KC>(p, batch, s);                                             \
    else launch_dma<AMV, DM_OC>(p, batch, s);
    if (am == DM_PK) { JAS_DMA_B(DM_PK) }
    else if (am == DM_KC) { JAS_DMA_B(DM_KC) }
    else { JAS_DMA_B(DM_OC) }
#undef JAS_DMA_B
    return true;
}

bool gemm_prefill_fused(int M, int N, int K, const void *A, const float *X, float *C, long ldc, const float *bias,
                        const DmaFused &fz, hipStream_t s)
{
    // SwiGLU: M virtual rows = 2 x the output features (gate / up tiles interleaved)
    if (fz.mode == FZ_SWIGLU && (M % 32 || !fz.A2 || bias)) return false;
    if (fz.mode == FZ_QKV && (fz.d % 16 || fz.dh % 16 || M != 3 * fz.d || !fz.pos || (fz.rope && !fz.rope_tab)))
        return false;
    const bool ok = gemm_dma(M, N, K, A, K, 1, X, 1, K, C, 1, ldc, bias, bias ? 1 : 0, JAS_ACT_NONE, 0, 1, 0, 0, 0, 0,
                             s, true, false, &fz);
    return ok && hipGetLastError() == hipSuccess;
}

jas_status gemm_general(int M, int N, int K, const void *A, long as0, long as1, const float *B, long bs0, long bs1,
                        float *C, long cs0, long cs1, const float *bias, int bias_mode, int act, int accumulate,
                        int batch, long abs_, long bbs, long cbs, long biasbs, hipStream_t s, bool a_packed,
                        bool a_bf16)
{
    JAS_CHECK(!a_bf16 || a_packed, JAS_ERR_INVALID, "gemm: bf16 A only in the packed layout");
    JAS_CHECK(!a_packed || (K % 16 == 0 && batch == 1), JAS_ERR_INVALID, "gemm: packed A needs K % 16 == 0");
    if (gemm_dma(M, N, K, A, as0, as1, B, bs0, bs1, C, cs0, cs1, bias, bias_mode, act, accumulate, batch, abs_, bbs,
                 cbs, biasbs, s, a_packed, a_bf16)) {
        JAS_LAUNCH_CHECK();
        return JAS_OK;
    }
    TileArgs p;
    p.A = (const float *)A; p.B = B; p.C = C; p.bias = bias_mode ? bias : nullptr;
    p.as0 = as0; p.as1 = as1; p.bs0 = bs0; p.bs1 = bs1; p.cs0 = cs0; p.cs1 = cs1;
    p.abs_ = abs_; p.bbs = bbs; p.cbs = cbs; p.biasbs = biasbs;
    p.M = M; p.N = N; p.K = K;
    p.bias_mode = bias_mode; p.act = act; p.accumulate = accumulate;
    JAS_CHECK(!a_packed || (K % 16 == 0 && batch == 1), JAS_ERR_INVALID, "gemm: packed A needs K % 16 == 0");
    int am = a_packed ? (a_bf16 ? LM_PKB : LM_PK) : pick_mode((const float *)A, as0, as1, M, K, abs_);
    int bm = pick_mode(B, bs1, bs0, N, K, bbs);
    bool c4 = cs0 == 1 && al16(C) && (cs1 % 4 == 0) && (cbs % 4 == 0);
    // 64-wide tiles when 128-wide ones give at most three workgroups per CU: too few to fill
    // the chip, or so few rounds that the last, partly empty one weighs (GPT-2-small prefill
    // GEMMs of 576 and 768 such workgroups: 8.34 -> 8.05 ms per prefill)
    const bool small = (long)ceil_div(N, TBN) * ceil_div(M, TBM) * batch <= 3 * 256;
    if (am == LM_PKB) launch_tile_b<LM_PKB>(p, bm, c4, small, batch, s);
    else if (am == LM_PK) launch_tile_b<LM_PK>(p, bm, c4, small, batch, s);
    else if (am == LM_KC) launch_tile_b<LM_KC>(p, bm, c4, small, batch, s);
    else if (am == LM_OC) launch_tile_b<LM_OC>(p, bm, c4, small, batch, s);
    else launch_tile_b<LM_GEN>(p, bm, c4, small, batch, s);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

// first maximum (ties to the lowest index) over the four 16-lane rows of a wave: lanes l,
// l ^ 16, l ^ 32, l ^ 48 end with the same pair (gfx950 permlane swaps, no LDS round trip)
__device__ __forceinline__ void argmax_rows(float &bv, int &bi)
{
    auto step = [&](bool rows32) {
        const unsigned vb = __float_as_uint(bv), ib = (unsigned)bi;
        const auto pv = rows32 ? __builtin_amdgcn_permlane32_swap(vb, vb, false, false)
                               : __builtin_amdgcn_permlane16_swap(vb, vb, false, false);
        const auto pi = rows32 ? __builtin_amdgcn_permlane32_swap(ib, ib, false, false)
                               : __builtin_amdgcn_permlane16_swap(ib, ib, false, false);
        float av = __uint_as_float(pv[0]), ov = __uint_as_float(pv[1]);
        int ai = (int)pi[0], oi = (int)pi[1];
        if (ov > av || (ov == av && oi < ai)) { av = ov; ai = oi; }
        bv = av;
        bi = ai;
    };
    step(true);
    step(false);
}

// ---------------------------------------------------------------- skinny (decode) GEMM
// One workgroup per row group of 16 rows (NT tiles of 16 rows for NT > 1; DUAL: tile 0 from
// W, tile 1 from W2 at the same 16 rows).  Its WPB waves interleave over the K chunks of 64
// and are reduced through LDS, then the fused epilogue runs.  No cross-workgroup reduction:
// on MI355X each XCD has its own L2, so a device-scope release/acquire inside the kernel
// would write back and invalidate L2 -- far costlier than the parallelism it buys.
//
// PACKED weights (weight_pack_offset): each wave-wide load is one contiguous 1 KB block
// holding exactly the A-operand float4s of 64 lanes, so a workgroup streams its rows as
// long contiguous runs instead of 16 rows x 64 B scattered 4*K bytes apart.
//
// WB (packed only): the weights are bf16 -- the same layout at 2 bytes per element, so one
// wave-wide load is a contiguous 512-byte block.  They feed v_mfma_f32_16x16x32_bf16
// directly: the activations are split exactly into three bf16 parts (x = hi + mid + lo,
// 8 significant bits each, so every bf16 x bf16 product is exact in fp32) and each weight
// fragment is multiplied by all three, accumulating in fp32.  The K order within a 32-wide
// step is permuted identically in both operands: slot j of lane group g is k = 16q + 4g + j
// for j < 4 (block q) and 16(q+1) + 4g + j - 4 for j >= 4 (block q+1) -- exactly what the
// packed weight and activation layouts put in that lane.  One such MFMA does the work of
// eight fp32 16x16x4 ones, so halving the weight bytes does not make the kernel
// matrix-core bound.
template <int NT, int WPB, int DEPTH, bool DUAL, bool PACKED, bool WB>
__global__ void __launch_bounds__(WPB * 64)
skinny_kernel(const void *__restrict__ W, const void *__restrict__ W2, const float *__restrict__ X, long ldx, int M,
              int N, int K, const SkinnyEpiArgs epi)
{
    static_assert(!WB || PACKED, "bf16 weights are packed");
    using WT = typename std::conditional<WB, uint16_t, float>::type;
    // one lane's weights of a 16-wide block (fp32) or of a 32-wide pair tile (bf16, slots 0-1)
    using WR = typename std::conditional<WB, u32x4, floatx4>::type;
    __shared__ floatx4 red[WPB][NT][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    // DUAL: tiles 0..NT/2-1 are gate rows, NT/2..NT-1 the up rows of the same 16-row blocks
    constexpr int NH = DUAL ? NT / 2 : NT;
    static_assert(!DUAL || NT % 2 == 0, "dual tiles come in (gate, up) pairs");
    const int m0 = blockIdx.x * NH * 16;
    const int K16 = K >> 4;

    const long RG = (M + 15) >> 4;  // row tiles of the packed layout
    const WT *wp[NT];
    long wrt[NT];  // packed: this tile's row-tile index
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const WT *base = (const WT *)((DUAL && t >= NH) ? W2 : W);
        const int tt = t % NH;  // 16-row block of this tile within the workgroup's rows
        if (PACKED) {
            // tiles past the last row tile (M not a multiple of NH*16) re-read the last one;
            // their rows are >= M and the epilogue discards them
            wrt[t] = min((long)(m0 / 16 + tt), RG - 1);
            wp[t] = base + lane * (WB ? 8 : 4);
        } else {
            int row = m0 + tt * 16 + r16;
            row = row < M ? row : M - 1;  // clamped rows are computed and discarded
            wp[t] = base + (long)row * K + 4 * g;
        }
    }
    // token rows >= N feed only output columns >= N, which the epilogue discards, so the
    // activation loads need no predicate (row 0 stands in for them)
    const float *xp = PACKED ? X + (long)lane * 4 : X + (long)(r16 < N ? r16 : 0) * ldx + 4 * g;

    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

    // K split (PARTIAL mode): this workgroup owns chunks [c_begin, c_end).  The streaming
    // loop covers the full 64-wide chunks; a partial last chunk (K % 64 != 0) is done once
    // at the end with predicated loads.
    const int c_begin = blockIdx.y * epi.cpb;
    const int c_end = min((K + 63) >> 6, c_begin + epi.cpb);
    const int c_full = min(K >> 6, c_end);
    // chunk index of this wave's i-th chunk: cs + i * WPB.  w is made wave-uniform so every
    // bound below is a scalar branch and the loads in the steady state carry no predicate
    // (a predicated load puts a branch around it, and the wait before the MFMAs then drains
    // the whole pipeline).
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int cs = c_begin + wu;
    const int nw = cs < c_full ? (c_full - cs + WPB - 1) / WPB : 0;
    WR wb[DEPTH][NT][4];
    float4 xb[DEPTH][4];
    const int K32 = k32_of(K);
    auto load = [&](int c, WR (&wv)[NT][4], float4 (&xv)[4]) {
        const int k = c * 64;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if constexpr (WB) {
                    if (q < 2)  // pair tiles 2c, 2c+1
                        wv[t][q] = __builtin_nontemporal_load(
                            (const u32x4 *)(wp[t] + weight_tile_offset_b(wrt[t], 2 * c + q, K32, RG)));
                } else if (PACKED)
                    wv[t][q] = __builtin_nontemporal_load(
                        (const floatx4 *)(wp[t] + weight_tile_offset(wrt[t], 4 * c + q, K16, RG)));
                else
                    wv[t][q] = __builtin_nontemporal_load((const floatx4 *)(wp[t] + k + 16 * q));
            }
            if (PACKED)  // contiguous 1 KB per wave
                xv[q] = *(const float4 *)(xp + (long)(4 * c + q) * 256);
            else
                xv[q] = *(const float4 *)(xp + k + 16 * q);
        }
    };
    auto compute = [&](const WR (&wv)[NT][4], const float4 (&xv)[4]) {
        if constexpr (WB) {
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {  // blocks 2pr, 2pr+1: one 32-wide MFMA step
                const float4 a = xv[2 * pr], b = xv[2 * pr + 1];
                const float x8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                bf16x8 xh, xm, xl;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const __bf16 h = (__bf16)x8[j];
                    const float r1 = x8[j] - (float)h;   // exact
                    const __bf16 m = (__bf16)r1;
                    const float r2 = r1 - (float)m;      // exact, at most 8 significant bits
                    xh[j] = h;
                    xm[j] = m;
                    xl[j] = (__bf16)r2;                  // exact
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const bf16x8 wf = __builtin_bit_cast(bf16x8, wv[t][pr]);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xl, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xm, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xh, acc[t], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t] = mfma4(wv[t][q][0], xv[q].x, acc[t]);
                    acc[t] = mfma4(wv[t][q][1], xv[q].y, acc[t]);
                    acc[t] = mfma4(wv[t][q][2], xv[q].z, acc[t]);
                    acc[t] = mfma4(wv[t][q][3], xv[q].w, acc[t]);
                }
        }
    };
#pragma unroll
    for (int j = 0; j < DEPTH - 1; ++j)
        if (j < nw) load(cs + j * WPB, wb[j], xb[j]);
    int i = 0;
    // steady state: DEPTH chunks per trip, every load in range
    for (; i + 2 * DEPTH - 2 < nw; i += DEPTH) {
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) {
            load(cs + (i + j + DEPTH - 1) * WPB, wb[(j + DEPTH - 1) % DEPTH], xb[(j + DEPTH - 1) % DEPTH]);
            compute(wb[j], xb[j]);
        }
    }
    // drain (i % DEPTH == 0 here, so the ring slots are compile-time indices)
#pragma unroll
    for (int j = 0; j < 2 * DEPTH - 1; ++j) {
        if (i + j < nw) {
            if (i + j + DEPTH - 1 < nw)
                load(cs + (i + j + DEPTH - 1) * WPB, wb[(j + DEPTH - 1) % DEPTH], xb[(j + DEPTH - 1) % DEPTH]);
            compute(wb[j % DEPTH], xb[j % DEPTH]);
        }
    }
    // partial last chunk: the wave whose stride reaches it; blocks (packed) or lanes
    // (row-major) past K read as zero
    if (c_full < c_end && (c_full - c_begin) % WPB == wu) {
        const int c = c_full, k = c * 64;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool in = PACKED ? (4 * c + q) < K16 : (k + 16 * q + 4 * g) < K;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if constexpr (WB) {
                    if (q % 2 == 0)  // a pair tile whose first block is in range (its padding is zero)
                        wb[0][t][q / 2] = in ? *(const u32x4 *)(wp[t] + weight_tile_offset_b(wrt[t], 2 * c + q / 2, K32, RG))
                                             : u32x4{0u, 0u, 0u, 0u};
                } else if (PACKED)
                    wb[0][t][q] = in ? *(const floatx4 *)(wp[t] + weight_tile_offset(wrt[t], 4 * c + q, K16, RG))
                                     : floatx4{0.f, 0.f, 0.f, 0.f};
                else
                    wb[0][t][q] = in ? *(const floatx4 *)(wp[t] + k + 16 * q) : floatx4{0.f, 0.f, 0.f, 0.f};
            }
            if (PACKED)
                xb[0][q] = in ? *(const float4 *)(xp + (long)(4 * c + q) * 256) : make_float4(0.f, 0.f, 0.f, 0.f);
            else
                xb[0][q] = in ? *(const float4 *)(xp + k + 16 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        compute(wb[0], xb[0]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) red[w][t][lane] = acc[t];
    __syncthreads();

    // epilogue: thread (t, ln) owns rows m..m+3 of tile t for token n = ln % 16
    const int n_items = NH * 64;
    const int t = tid / 64, ln = tid % 64;
    const int n = ln & 15;
    const int m = m0 + t * 16 + 4 * (ln >> 4);
    const bool live = tid < n_items && n < N && m < M;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    const int nv = live ? min(4, M - m) : 0;
    if (live) {
        floatx4 s0 = red[0][t][ln];
#pragma unroll
        for (int ww = 1; ww < WPB; ++ww) s0 += red[ww][t][ln];
        v[0] = s0[0], v[1] = s0[1], v[2] = s0[2], v[3] = s0[3];
    }
    if constexpr (!DUAL) {
        if (epi.amax_v) {  // first maximum of the stored values over this workgroup's rows
            __shared__ float sbv[NH * 16];
            __shared__ int sbi[NH * 16];
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            for (int r = 0; r < nv; ++r) {
                float x = epi.bias ? v[r] + epi.bias[m + r] : v[r];
                x = apply_act(x, epi.act);
                if (x > bv) { bv = x; bi = m + r; }
            }
            // the four lanes of a token in each wave (ln, ln ^ 16, ln ^ 32, ln ^ 48) combine in
            // registers, then the tile waves' winners through LDS (ties to the lowest index)
            argmax_rows(bv, bi);
            if (tid < n_items && ln < 16) { sbv[t * 16 + ln] = bv; sbi[t * 16 + ln] = bi; }
            __syncthreads();
            if (tid < 16) {
                for (int k = 1; k < NH; ++k) {
                    const float ov = sbv[k * 16 + tid];
                    const int oi = sbi[k * 16 + tid];
                    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
                }
                epi.amax_v[(long)tid * gridDim.x + blockIdx.x] = bv;
                epi.amax_i[(long)tid * gridDim.x + blockIdx.x] = bi;
            }
        }
    }
    if (!live) return;

    if (epi.mode == EPI_PARTIAL) {  // raw split-K partial, [split][16][M]; the consumer reduces
        float *o = epi.out + ((long)blockIdx.y * 16 + n) * M + m;
        if (nv == 4 && (M & 3) == 0) *(float4 *)o = make_float4(v[0], v[1], v[2], v[3]);
        else
            for (int r = 0; r < nv; ++r) o[r] = v[r];
        return;
    }
    if constexpr (DUAL) {  // SwiGLU: silu(gate) * up
        floatx4 s1 = red[0][t + NH][ln];
#pragma unroll
        for (int ww = 1; ww < WPB; ++ww) s1 += red[ww][t + NH][ln];
        if (epi.out_packed && nv == 4) {
            *(float4 *)(epi.out + packed_b_offset(n, m)) =
                make_float4(silu_f(v[0]) * s1[0], silu_f(v[1]) * s1[1], silu_f(v[2]) * s1[2], silu_f(v[3]) * s1[3]);
            return;
        }
        float *o = epi.out + (long)n * epi.ldo + m;
        for (int r = 0; r < nv; ++r) o[r] = silu_f(v[r]) * s1[r];
        return;
    } else {
        if (epi.bias)
            for (int r = 0; r < nv; ++r) v[r] = v[r] + epi.bias[m + r];
        if (epi.mode == EPI_STORE) {
            if (epi.out_packed && nv == 4) {
                *(float4 *)(epi.out + packed_b_offset(n, m)) = make_float4(
                    apply_act(v[0], epi.act), apply_act(v[1], epi.act), apply_act(v[2], epi.act), apply_act(v[3], epi.act));
                return;
            }
            float *o = epi.out + (long)n * epi.ldo + m;
            for (int r = 0; r < nv; ++r) o[r] = apply_act(v[r], epi.act);
        } else if (epi.mode == EPI_RESID) {
            float *o = epi.out + (long)n * epi.ldo + m;
            for (int r = 0; r < nv; ++r) o[r] = o[r] + v[r];
        } else {  // EPI_QKV (m % 4 == 0, d % 16 == 0, dh even: the 4 rows share a section and head)
            const int sec = m / epi.d, e = m - sec * epi.d, h = e / epi.dh, ee = e - h * epi.dh;
            const int pos = epi.pos[n];
            if (epi.rope && sec < 2) {
#pragma unroll
                for (int pr = 0; pr < 2; ++pr) {
                    int i = (ee + 2 * pr) / 2;
                    double cs, sn;
                    if (epi.rope_tab) {
                        const double2 cst = epi.rope_tab[(long)pos * (epi.dh / 2) + i];
                        cs = cst.x, sn = cst.y;
                    } else {
                        const double a = (double)pos * pow((double)epi.theta, -2.0 * i / (double)epi.dh);
                        cs = cos(a), sn = sin(a);
                    }
                    double x0 = v[2 * pr], x1 = v[2 * pr + 1];
                    v[2 * pr] = (float)(x0 * cs - x1 * sn);
                    v[2 * pr + 1] = (float)(x0 * sn + x1 * cs);
                }
            }
            if (sec == 0) {
                *(float4 *)(epi.q_out + (long)n * epi.d + e) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                const long ce = (long)n * epi.kv_sb + (long)h * epi.kv_sh + (long)pos * epi.dh + ee;
                float *cache = sec == 1 ? epi.k_cache : epi.v_cache;
                if (epi.kv_bf16)
                    *(u32x2 *)((uint16_t *)cache + ce) =
                        u32x2{(uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                              (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16)};
                else
                    *(float4 *)(cache + ce) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

template <int NT, int WPB, int DEPTH, bool DUAL, bool PACKED, bool WB = false>
static void launch_skinny(const void *W, const void *W2, const float *X, long ldx, int M, int N, int K,
                          const SkinnyEpiArgs &epi, hipStream_t s)
{
    const int rows = DUAL ? 16 * (NT / 2) : NT * 16;
    const int ks = epi.mode == EPI_PARTIAL ? std::max(1, epi.ksplit) : 1;
    hipLaunchKernelGGL((skinny_kernel<NT, WPB, DEPTH, DUAL, PACKED, WB>), dim3((M + rows - 1) / rows, ks),
                       dim3(WPB * 64), 0, s, W, W2, X, ldx, M, N, K, epi);
}

// Geometry per decode shape, from a cold-weight sweep on MI355X (16 tokens, packed weights).
// More row tiles per workgroup amortise each activation chunk (read from L2) over more
// weight bytes, best when the workgroup count lands on the 256 CUs (the QKV projection:
// three tiles); small matrices (GPT-2 widths) are latency-bound and keep one tile and
// 8 waves so that more workgroups are in flight.
SkinnyTuning skinny_default_tuning(int M, int K, bool dual, bool split, bool wbf16)
{
    SkinnyTuning t;
    const int rt = (M + 15) / 16;
    if (wbf16) {  // bf16 weights (cold-weight sweep): half the bytes per tile, deeper rings
        if (dual && rt >= 512) { t.nt = 6; t.wpb = 4; t.depth = 2; }  // one round (fp32 note below)
        else if (dual) { t.nt = 2; t.wpb = 4; t.depth = 3; }
        else if (split && rt >= 256) {
            if (K >= 8192) { t.nt = 4; t.wpb = 4; t.depth = 4; }
            else { t.nt = 2; t.wpb = 8; t.depth = 2; }
        } else if (split) { t.nt = 2; t.wpb = 8; t.depth = 2; }
        else if (rt >= 1536 && K >= 2048) { t.nt = 4; t.wpb = 4; t.depth = 2; }
        else if (rt >= 1536) { t.nt = 4; t.wpb = 4; t.depth = 3; }
        else if (rt >= 512) { t.nt = 3; t.wpb = 4; t.depth = 4; }
        else { t.nt = 1; t.wpb = 8; t.depth = 3; }
        return t;
    }
    if (dual) {                      // SwiGLU gate/up pairs
        // three pairs per workgroup at LLaMA-7B width: 688 row tiles in 230 workgroups, one
        // round on 256 CUs instead of 2.7 (236 VGPRs; one 4-wave workgroup per CU keeps
        // ~100 KB in flight): GEMM time per step -4 %.  One pair otherwise.
        if (rt >= 512) { t.nt = 6; t.wpb = 4; t.depth = 2; }
        else { t.nt = 2; t.wpb = 4; t.depth = 3; }
    } else if (split) {              // split-K residual projections
        // (two tiles: four would need twice the K splits, and the norm kernel that sums
        // the split partials then reads twice as much)
        if (rt >= 256) { t.nt = 2; t.wpb = 4; t.depth = K >= 8192 ? 2 : 3; }
        else { t.nt = 2; t.wpb = 8; t.depth = 2; }
    } else if (rt >= 1536) {         // LM head (short K: more waves share each row tile's chunks)
        if (K >= 2048) { t.nt = 4; t.wpb = 4; t.depth = 3; }
        else { t.nt = 2; t.wpb = 8; t.depth = 2; }
    } else if (rt >= 512) {          // QKV at LLaMA-7B width: 768 row tiles, 3 per workgroup
        t.nt = 3; t.wpb = 4; t.depth = 2;  // = 256 workgroups, one per CU (4 tiles: 192, 15 % slower)
    } else {
        t.nt = 1; t.wpb = 8; t.depth = 3;
    }
    return t;
}

// K splits of a split-K residual projection: enough splits for about 256 workgroups with
// the split geometry above, at most 8 and at least two 64-wide chunks per split
int skinny_row_groups(int M, int K, bool dual, bool split, bool wbf16)
{
    const SkinnyTuning tu = skinny_default_tuning(M, K, dual, split, wbf16);
    const int nt = dual && (tu.nt < 2 || tu.nt % 2) ? 2 : tu.nt;
    const int rows = (dual ? nt / 2 : nt) * 16;
    return (M + rows - 1) / rows;
}

int skinny_pick_ksplit(int M, int K, bool wbf16)
{
    const int nt = skinny_default_tuning(M, K, false, true, wbf16).nt;
    const int wgs = ((M + 15) / 16 + nt - 1) / nt, nchunk = (K + 63) / 64;
    int ks = std::max(1, std::min({(256 + wgs - 1) / wgs, nchunk / 2, 8}));
    const int cpb = (nchunk + ks - 1) / ks;
    return (nchunk + cpb - 1) / cpb;  // every split non-empty
}

jas_status skinny_gemm(const void *W, const void *W2, const float *X, long ldx, int M, int N, int K,
                       const SkinnyEpiArgs &epi, hipStream_t s, bool packed, const SkinnyTuning *tune, bool wbf16)
{
    JAS_CHECK(!wbf16 || packed, JAS_ERR_INVALID, "skinny_gemm: bf16 weights only in the packed layout");
    JAS_CHECK(N >= 1 && N <= 16 && M > 0 && K > 0 && K % 4 == 0 && ldx % 4 == 0, JAS_ERR_INVALID,
              "skinny_gemm: unsupported shape");
    JAS_CHECK(!packed || K % 16 == 0, JAS_ERR_INVALID, "skinny_gemm: packed weights need K % 16 == 0");
    JAS_CHECK(!epi.out_packed || (M % 16 == 0 && (epi.mode == EPI_STORE || epi.mode == EPI_SWIGLU)), JAS_ERR_INVALID,
              "skinny_gemm: packed output needs M % 16 == 0");
    JAS_CHECK(al16(W) && al16(X) && (!W2 || al16(W2)), JAS_ERR_INVALID, "skinny_gemm: operands must be 16B aligned");
    const bool dual = epi.mode == EPI_SWIGLU;
    if (epi.mode == EPI_QKV)
        JAS_CHECK(epi.d % 16 == 0 && epi.dh % 4 == 0 && M == 3 * epi.d, JAS_ERR_INVALID, "skinny_gemm: bad QKV shape");
    if (dual) JAS_CHECK(W2 != nullptr, JAS_ERR_INVALID, "skinny_gemm: SwiGLU needs both weights");
    SkinnyTuning tu = tune ? *tune : skinny_default_tuning(M, K, dual, epi.mode == EPI_PARTIAL, wbf16);
    if (!tune && !packed && tu.nt > 2) tu.nt = 2;  // more tiles: packed weights only
    const int nt = dual && (tu.nt < 2 || tu.nt % 2) ? 2 : tu.nt;
    SkinnyEpiArgs ep = epi;
    const int nchunk = (K + 63) / 64;
    if (ep.mode == EPI_PARTIAL) {
        JAS_CHECK(!dual && ep.ksplit >= 1 && ep.out, JAS_ERR_INVALID, "skinny_gemm: bad split-K partial request");
        ep.cpb = (nchunk + ep.ksplit - 1) / ep.ksplit;
        ep.ksplit = (nchunk + ep.cpb - 1) / ep.cpb;  // splits actually used (all non-empty)
        JAS_CHECK(ep.ksplit == epi.ksplit, JAS_ERR_INVALID, "skinny_gemm: K too short for the requested split");
    } else {
        ep.cpb = nchunk;
        ep.ksplit = 1;
    }
#define JAS_SK(NTV, WPBV, DV, PV, DEP)                                                         \
    if (nt == NTV && tu.wpb == WPBV && dual == DV && packed == PV && tu.depth == DEP) {       \
        launch_skinny<NTV, WPBV, DEP, DV, PV>(W, W2, X, ldx, M, N, K, ep, s);                 \
        JAS_LAUNCH_CHECK();                                                                    \
        return JAS_OK;                                                                         \
    }
#define JAS_SK_D(NTV, WPBV, DV, PV) JAS_SK(NTV, WPBV, DV, PV, 2) JAS_SK(NTV, WPBV, DV, PV, 3) JAS_SK(NTV, WPBV, DV, PV, 4)
#define JAS_SK_P(NTV, WPBV, DV) JAS_SK_D(NTV, WPBV, DV, true) JAS_SK_D(NTV, WPBV, DV, false)
    if (wbf16) {  // the geometries the default tuning picks
#define JAS_SKB(NTV, WPBV, DV, DEP)                                                           \
    if (nt == NTV && tu.wpb == WPBV && dual == DV && tu.depth == DEP) {                      \
        launch_skinny<NTV, WPBV, DEP, DV, true, true>(W, W2, X, ldx, M, N, K, ep, s);         \
        JAS_LAUNCH_CHECK();                                                                    \
        return JAS_OK;                                                                         \
    }
        JAS_SKB(2, 4, true, 3) JAS_SKB(2, 4, true, 4) JAS_SKB(2, 4, false, 2) JAS_SKB(2, 4, false, 3)
        JAS_SKB(2, 4, false, 4) JAS_SKB(2, 8, false, 2) JAS_SKB(2, 8, false, 3) JAS_SKB(4, 4, false, 2)
        JAS_SKB(4, 4, false, 3) JAS_SKB(4, 4, false, 4) JAS_SKB(1, 8, false, 3) JAS_SKB(1, 8, false, 4)
        JAS_SKB(3, 4, false, 3) JAS_SKB(3, 4, false, 4) JAS_SKB(6, 4, true, 2)
#undef JAS_SKB
        return fail(JAS_ERR_INVALID, "skinny_gemm: unsupported tuning for bf16 weights");
    }
    JAS_SK_P(1, 4, false) JAS_SK_P(1, 8, false) JAS_SK_P(2, 4, false) JAS_SK_P(2, 8, false) JAS_SK_P(2, 4, true)
    JAS_SK_P(2, 8, true)
    // 1024-thread workgroups get 128 VGPRs: depth 4 would spill
    JAS_SK(1, 16, false, true, 2) JAS_SK(1, 16, false, true, 3) JAS_SK(1, 16, false, false, 2)
    JAS_SK(1, 16, false, false, 3)
    // four row tiles per workgroup share each activation chunk (packed weights only)
    JAS_SK(4, 4, false, true, 2) JAS_SK(4, 4, false, true, 3) JAS_SK(4, 8, false, true, 2)
    JAS_SK(3, 4, false, true, 2) JAS_SK(3, 4, false, true, 3) JAS_SK(3, 8, false, true, 2)
    // dual with three (gate, up) pairs per workgroup (packed weights only)
    JAS_SK(6, 4, true, true, 2)
#undef JAS_SK_P
#undef JAS_SK_D
#undef JAS_SK
    return fail(JAS_ERR_INVALID, "skinny_gemm: unsupported tuning");
}

// ---------------------------------------------------------------- packed weight layout
// BF: the bf16 pair-tile layout (weight_pack_offset_b), K padded to a multiple of 32
template <bool BF>
__global__ void weight_pack_kernel(const void *__restrict__ src, void *__restrict__ dst, int M, int Mp, int K,
                                   int unpack)
{
    long p = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= (long)Mp * (BF ? k32_of(K) : K)) return;
    int r, k;
    if (BF) weight_pack_coords_b(p, K, Mp >> 4, &r, &k);
    else weight_pack_coords(p, K, Mp >> 4, &r, &k);
    const bool real = r < M && k < K;
    if (unpack) {
        const float v = BF ? bf16_to_f32(((const uint16_t *)src)[p]) : ((const float *)src)[p];
        if (real) ((float *)dst)[(long)r * K + k] = v;
    } else {
        const float v = real ? ((const float *)src)[(long)r * K + k] : 0.0f;
        if (BF) ((uint16_t *)dst)[p] = f32_to_bf16(v);
        else ((float *)dst)[p] = v;
    }
}

template <bool BF>
__global__ void fill_normal_packed_kernel(void *x, int M, int Mp, int K, uint64_t key, float mean, float std)
{
    long stride = (long)gridDim.x * blockDim.x;
    for (long p = (long)blockIdx.x * blockDim.x + threadIdx.x; p < (long)Mp * (BF ? k32_of(K) : K); p += stride) {
        int r, k;
        if (BF) weight_pack_coords_b(p, K, Mp >> 4, &r, &k);
        else weight_pack_coords(p, K, Mp >> 4, &r, &k);
        float v = 0.0f;
        if (r < M && k < K) {
            uint64_t i = (uint64_t)r * K + k;  // the row-major element index drives the generator
            uint64_t a = splitmix64(key + 2 * i), b = splitmix64(key + 2 * i + 1);
            double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
            double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
            double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
            v = (float)((double)mean + (double)std * z);
        }
        if (BF) ((uint16_t *)x)[p] = f32_to_bf16(v);
        else ((float *)x)[p] = v;
    }
}

jas_status weight_pack(const void *src, void *dst, int M, int K, bool unpack, hipStream_t s, bool bf16)
{
    JAS_CHECK(K % 16 == 0, JAS_ERR_INVALID, "weight_pack: K must be a multiple of 16");
    const int Mp = (M + 15) / 16 * 16;
    long n = (long)Mp * (bf16 ? k32_of(K) : K);
    if (bf16)
        hipLaunchKernelGGL(weight_pack_kernel<true>, dim3(ceil_div(n, 256)), dim3(256), 0, s, src, dst, M, Mp, K,
                           unpack ? 1 : 0);
    else
        hipLaunchKernelGGL(weight_pack_kernel<false>, dim3(ceil_div(n, 256)), dim3(256), 0, s, src, dst, M, Mp, K,
                           unpack ? 1 : 0);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

jas_status fill_normal_packed(void *x, int M, int K, uint64_t seed, uint64_t stream_id, float mean, float std,
                              hipStream_t s, bool bf16)
{
    JAS_CHECK(K % 16 == 0, JAS_ERR_INVALID, "fill_normal_packed: K must be a multiple of 16");
    const int Mp = (M + 15) / 16 * 16;
    unsigned nb = (unsigned)std::min<long>(((long)Mp * (bf16 ? k32_of(K) : K) + 255) / 256, 65536);
    if (bf16)
        hipLaunchKernelGGL(fill_normal_packed_kernel<true>, dim3(nb), dim3(256), 0, s, x, M, Mp, K,
                           stream_key(seed, stream_id), mean, std);
    else
        hipLaunchKernelGGL(fill_normal_packed_kernel<false>, dim3(nb), dim3(256), 0, s, x, M, Mp, K,
                           stream_key(seed, stream_id), mean, std);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

// ---------------------------------------------------------------- fp64 GEMM
// 64x64 tile, K step 8, 256 threads (4 waves as 2x2 of 32x32): v_mfma_f64_16x16x4_f64 with
// A[i = l%16][k = l/16], B[k = l/16][j = l%16]; result register r of lane l holds
// D[i = l/16 + 4r][j = l%16] (the fp64 form interleaves rows, unlike the fp32 16x16x4).
typedef double doublex4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256)
gemm_f64_kernel(int M, int N, int K, const double *__restrict__ A, long as0, long as1, const double *__restrict__ B,
                long bs0, long bs1, double *__restrict__ C, long cs0, long cs1, const double *__restrict__ bias,
                int bias_mode)
{
    __shared__ double As[64][9];
    __shared__ double Bs[64][9];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    doublex4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = doublex4{0.0, 0.0, 0.0, 0.0};
    for (int k0 = 0; k0 < K; k0 += 8) {
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 2; ++q) {  // 64 x 8 tiles of A and B, 512 elements each
            int idx = tid + q * 256, o = idx >> 3, k = idx & 7;
            int gm = m0 + o, gn = n0 + o, gk = k0 + k;
            As[o][k] = (gm < M && gk < K) ? A[(long)gm * as0 + (long)gk * as1] : 0.0;
            Bs[o][k] = (gn < N && gk < K) ? B[(long)gk * bs0 + (long)gn * bs1] : 0.0;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 8; kk += 4)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(As[wm * 32 + i * 16 + r16][kk + g],
                                                                     Bs[wn * 32 + j * 16 + r16][kk + g], acc[i][j], 0,
                                                                     0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int m = m0 + wm * 32 + i * 16 + g + 4 * r, n = n0 + wn * 32 + j * 16 + r16;
                if (m >= M || n >= N) continue;
                double v = acc[i][j][r];
                if (bias_mode == 1) v = v + bias[m];
                else if (bias_mode == 2) v = v + bias[n];
                C[(long)m * cs0 + (long)n * cs1] = v;
            }
}

} // namespace jas

using namespace jas;

extern "C" jas_status jas_gemm_f64(int M, int N, int K, const double *A, long as0, long as1, const double *B, long bs0,
                                   long bs1, double *C, long cs0, long cs1, const double *bias, int bias_mode,
                                   jas_stream_t stream)
{
    JAS_CHECK(M >= 0 && N >= 0 && K >= 0 && A && B && C, JAS_ERR_INVALID, "jas_gemm_f64: bad arguments");
    JAS_CHECK(bias_mode >= 0 && bias_mode <= 2 && (bias_mode == 0 || bias), JAS_ERR_INVALID, "jas_gemm_f64: bad bias");
    if (M == 0 || N == 0) return JAS_OK;
    hipLaunchKernelGGL(gemm_f64_kernel, dim3(ceil_div(N, 64), ceil_div(M, 64)), dim3(256), 0, stream_or_default(stream),
                       M, N, K, A, as0, as1, B, bs0, bs1, C, cs0, cs1, bias, bias_mode);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}

extern "C" jas_status jas_gemm(int M, int N, int K, const float *A, long as0, long as1, const float *B, long bs0,
                               long bs1, float *C, long cs0, long cs1, const float *bias, int bias_mode, int act,
                               int accumulate, int batch, long abs_, long bbs, long cbs, long biasbs,
                               jas_stream_t stream)
{
    JAS_CHECK(M >= 0 && N >= 0 && K >= 0 && batch >= 1, JAS_ERR_INVALID, "jas_gemm: negative size");
    JAS_CHECK(A && B && C, JAS_ERR_INVALID, "jas_gemm: null operand");
    JAS_CHECK(bias_mode >= 0 && bias_mode <= 2 && (bias_mode == 0 || bias), JAS_ERR_INVALID, "jas_gemm: bad bias");
    JAS_CHECK(act >= JAS_ACT_NONE && act <= JAS_ACT_SIGMOID, JAS_ERR_INVALID, "jas_gemm: bad activation");
    if (M == 0 || N == 0) return JAS_OK;
    hipStream_t s = stream_or_default(stream);
    // decode shape: weights [M][K] row-major, tokens K-contiguous, token-major output
    if (batch == 1 && N <= 16 && as1 == 1 && bs0 == 1 && cs0 == 1 && K % 4 == 0 && as0 == K && bs1 % 4 == 0 &&
        al16(A) && al16(B) && bias_mode != 2 && !accumulate && K > 0) {
        SkinnyEpiArgs e;
        e.mode = EPI_STORE;
        e.act = act;
        e.bias = bias_mode == 1 ? bias : nullptr;
        e.out = C;
        e.ldo = cs1;
        return skinny_gemm(A, nullptr, B, bs1, M, N, K, e, s, false, nullptr);
    }
    return gemm_general(M, N, K, A, as0, as1, B, bs0, bs1, C, cs0, cs1, bias, bias_mode, act, accumulate, batch, abs_,
                        bbs, cbs, biasbs, s, false);
}

// C(m, n) += R(m, n) after a product that did not take the residual in its epilogue
__global__ void add_residual_kernel(float *C, long cs0, long cs1, const float *R, long rs0, long rs1, int M, int N)
{
    const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (long)M * N) return;
    const int m = (int)(g / N), n = (int)(g % N);
    float *c = C + (long)m * cs0 + (long)n * cs1;
    *c = *c + R[(long)m * rs0 + (long)n * rs1];
}

extern "C" jas_status jas_gemm_residual(int M, int N, int K, const float *A, long as0, long as1, const float *B,
                                        long bs0, long bs1, float *C, long cs0, long cs1, const float *bias,
                                        int bias_mode, int act, const float *R, long rs0, long rs1,
                                        jas_stream_t stream)
{
    JAS_CHECK(M >= 0 && N >= 0 && K >= 0, JAS_ERR_INVALID, "jas_gemm_residual: negative size");
    JAS_CHECK(A && B && C && R, JAS_ERR_INVALID, "jas_gemm_residual: null operand");
    JAS_CHECK(bias_mode >= 0 && bias_mode <= 2 && (bias_mode == 0 || bias), JAS_ERR_INVALID,
              "jas_gemm_residual: bad bias");
    JAS_CHECK(act >= JAS_ACT_NONE && act <= JAS_ACT_SIGMOID, JAS_ERR_INVALID, "jas_gemm_residual: bad activation");
    if (M == 0 || N == 0) return JAS_OK;
    hipStream_t s = stream_or_default(stream);
    if (gemm_dma(M, N, K, A, as0, as1, B, bs0, bs1, C, cs0, cs1, bias, bias_mode, act, 0, 1, 0, 0, 0, 0, s, false,
                 false, nullptr, R, rs0, rs1)) {
        JAS_LAUNCH_CHECK();
        return JAS_OK;
    }
    // other operand layouts: the product, then the residual added in the same order
    const jas_status st = jas_gemm(M, N, K, A, as0, as1, B, bs0, bs1, C, cs0, cs1, bias, bias_mode, act, 0, 1, 0, 0,
                                   0, 0, stream);
    if (st != JAS_OK) return st;
    const long n = (long)M * N;
    hipLaunchKernelGGL(add_residual_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, C, cs0, cs1, R, rs0,
                       rs1, M, N);
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}
